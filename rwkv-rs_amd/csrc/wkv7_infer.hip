// WKV7 slot-mapped inference (decode / prefill) for gfx950, forward only.
//
// Semantics: /root/reference/crates/rwkv-nn/src/kernels/wkv7_infer/kernel.rs:15-114
// (wkv7_infer_forward_kernel). Active row b works on state slot batch_ids[b]
// of a [full_batch, H, 64, 64] fp32 state buffer, read and written in place
// (kernel.rs:27-42, 103-113). A step whose context_mask entry is 0 writes
// y = 0 and leaves the state untouched (kernel.rs:57-62). With use_dither the
// decay gets deterministic_dither(elapsed_t[slot] + valid_t) added, where
// valid_t counts the unmasked steps of this call before the current one
// (kernel.rs:8-13, 73-77). The state is always fp32 here; the reference's
// dither is tied to a reduced-precision state element type, so callers that
// want its arithmetic pass use_dither explicitly.
//
// Design: the forward kernel's thread layout and per-step arithmetic (one
// workgroup per (active row, head), a 2x4 state block per thread in VGPRs,
// operands from LDS). At T = 1 the kernel is bound by the 16 KiB state read
// and 16 KiB state write per (row, head): every thread moves two 16-byte rows
// each way, and the grid has Ba*H workgroups.
#include "wkv7_device.hpp"
#include "wkv7_launch.hpp"

namespace wkv7 {
namespace {

// Timesteps staged per LDS tile: 16 for prefill; 1 for a single decode step,
// where the small LDS footprint lets three workgroups share a CU (the step is
// bound by the HBM latency of its state read, so workgroups in flight count).
enum { V_W = 0, V_R, V_K, V_V, V_A, V_B, V_COUNT };


__device__ __forceinline__ float dither_f(uint32_t seed) {
  const uint32_t mixed = seed * 2654435769u;          // wrapping u32 product
  return (float)(int32_t)mixed * 4.547473508864641e-13f;   // 2^-41
}

template <typename Tin>
struct InferParams {
  const Tin *w, *r, *k, *v, *a, *b;
  const int32_t* batch_ids;
  float* state;
  const Tin* mask;
  const int32_t* elapsed_t;
  Tin* y;
  int T, H, full_batch, use_dither;
};

template <typename Tin>
__device__ __forceinline__ bool mask_on(const Tin* m, int64_t i);
template <>
__device__ __forceinline__ bool mask_on<float>(const float* m, int64_t i) { return m[i] != 0.0f; }
template <>
__device__ __forceinline__ bool mask_on<bf16_t>(const bf16_t* m, int64_t i) {
  return (m[i] & 0x7fffu) != 0u;   // +0 and -0 are "masked"
}

template <typename Tin, int kTile>
__global__ __launch_bounds__(kThreads) void wkv7_infer_kernel(InferParams<Tin> p) {
  __shared__ float4 tile[2][V_COUNT][kTile][16];   // 1.5 KiB per step
  __shared__ float ost[2][kTile][kHead];           // 0.5 KiB per step
  __shared__ int live[2][kTile];                   // step not masked

  const int h = blockIdx.x, bi = blockIdx.y;
  const int tid = threadIdx.x;
  const int L = tid & 15, q = tid >> 4;   // columns 4L.., row pair 2q, 2q+1
  const int up = (L >> 3) & 1;
  const int ro = 2 * q + up, rt = 2 * q + 1 - up;   // own and other row
  const int sl = (tid >> 4) & 15, pp = tid & 15;   // staging (threads 0..255)
  const bool stager = tid < 16 * kTile;

  const int T = p.T;
  const int64_t slot = p.batch_ids[bi];
  // An out-of-range slot would read and write outside the state buffer. The
  // host cannot see device-resident batch_ids, so the kernel refuses such a
  // row: its output is zeroed and no state is touched.
  if (slot < 0 || slot >= p.full_batch) {
    for (int64_t i = tid; i < (int64_t)T * kHead; i += kThreads) {
      const int64_t t = i / kHead, n = i % kHead;
      p.y[((int64_t)bi * T + t) * p.H * kHead + (int64_t)h * kHead + n] = Tin(0);
    }
    return;
  }
  const uint32_t elapsed = p.elapsed_t ? (uint32_t)p.elapsed_t[slot] : 0u;
  const int64_t tstride = (int64_t)p.H * kHead;
  const int64_t tok0 = ((int64_t)bi * T * p.H + h) * kHead;

  float* st = p.state + (slot * p.H + h) * (kHead * kHead) + 4 * L;
  float So[4], St[4];   // own and other row
  {
    const float4 x0 = *reinterpret_cast<const float4*>(st + ro * kHead);
    const float4 x1 = *reinterpret_cast<const float4*>(st + rt * kHead);
    So[0] = x0.x; So[1] = x0.y; So[2] = x0.z; So[3] = x0.w;
    St[0] = x1.x; St[1] = x1.y; St[2] = x1.z; St[3] = x1.w;
  }

  typedef Io<Tin> io;
  typename io::raw pre[V_COUNT];
  uint32_t valid_before_tile = 0;
  bool pre_live = true;
  uint32_t pre_vt = 0;   // unmasked steps before this thread's staged step

  auto gload = [&](int t0) {
    const int t = t0 + sl;
    if (stager && t < T) {
      pre_live = !p.mask || mask_on<Tin>(p.mask, (int64_t)bi * T + t);
      uint32_t vt = valid_before_tile;
      if (p.mask) {
        for (int u = t0; u < t; ++u) vt += mask_on<Tin>(p.mask, (int64_t)bi * T + u) ? 1u : 0u;
      } else {
        vt += (uint32_t)(t - t0);
      }
      pre_vt = vt;
      const int64_t off = tok0 + (int64_t)t * tstride + 4 * pp;
      pre[V_W] = io::load(p.w + off);
      pre[V_R] = io::load(p.r + off);
      pre[V_K] = io::load(p.k + off);
      pre[V_V] = io::load(p.v + off);
      pre[V_A] = io::load(p.a + off);
      pre[V_B] = io::load(p.b + off);
    }
  };
  auto lstore = [&](int buf, int t0) {
    if (stager && t0 + sl < T) {
      float4 x = io::widen(pre[V_W]);
      const float dith = p.use_dither ? dither_f(elapsed + pre_vt) : 0.0f;
      x.x = decay_f(sigmoid_f(x.x)) + dith;
      x.y = decay_f(sigmoid_f(x.y)) + dith;
      x.z = decay_f(sigmoid_f(x.z)) + dith;
      x.w = decay_f(sigmoid_f(x.w)) + dith;
      tile[buf][V_W][sl][pp] = x;
      tile[buf][V_R][sl][pp] = io::widen(pre[V_R]);
      tile[buf][V_K][sl][pp] = io::widen(pre[V_K]);
      tile[buf][V_V][sl][pp] = io::widen(pre[V_V]);
      tile[buf][V_A][sl][pp] = io::widen(pre[V_A]);
      tile[buf][V_B][sl][pp] = io::widen(pre[V_B]);
      if (pp == 0) live[buf][sl] = pre_live ? 1 : 0;
    }
  };
  auto count_live = [&](int t0, int nst) {
    if (!p.mask) return (uint32_t)nst;
    uint32_t n = 0;
    for (int u = 0; u < nst; ++u) n += mask_on<Tin>(p.mask, (int64_t)bi * T + t0 + u) ? 1u : 0u;
    return n;
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
    valid_before_tile += count_live(t0, nst);
    if (ti + 1 < ntiles) gload(t0 + kTile);

    for (int s = 0; s < nst; ++s) {
      float y = 0.0f;
      if (live[buf][s]) {   // uniform across the workgroup
        const float2 v2 = reinterpret_cast<const float2*>(tile[buf][V_V][s])[q];
        float sa_o, sa_t, y_t;
        fwd_step(So, St, tile[buf][V_W][s][L], tile[buf][V_A][s][L], tile[buf][V_B][s][L],
                 tile[buf][V_K][s][L], tile[buf][V_R][s][L],
                 up ? make_float2(v2.y, v2.x) : v2, sa_o, sa_t, y, y_t);
        row_pair_sum(y, y_t);   // y of the own row
      }
      if ((L & 7) == 0) ost[buf][s][ro] = y;
    }

    if (ti + 1 < ntiles) lstore(buf ^ 1, t0 + kTile);
    __syncthreads();
    if (stager && sl < nst) {
      const int64_t off = tok0 + (int64_t)(t0 + sl) * tstride + 4 * pp;
      io::store(p.y + off, reinterpret_cast<const float4*>(ost[buf][sl])[pp]);
    }
  }

  *reinterpret_cast<float4*>(st + ro * kHead) = make_float4(So[0], So[1], So[2], So[3]);
  *reinterpret_cast<float4*>(st + rt * kHead) = make_float4(St[0], St[1], St[2], St[3]);
}

template <typename Tin>
hipError_t launch_infer_t(const InferDesc& d, hipStream_t stream) {
  InferParams<Tin> p;
  p.w = static_cast<const Tin*>(d.w);
  p.r = static_cast<const Tin*>(d.r);
  p.k = static_cast<const Tin*>(d.k);
  p.v = static_cast<const Tin*>(d.v);
  p.a = static_cast<const Tin*>(d.a);
  p.b = static_cast<const Tin*>(d.b);
  p.batch_ids = d.batch_ids;
  p.state = d.state;
  p.mask = static_cast<const Tin*>(d.context_mask);
  p.elapsed_t = d.elapsed_t;
  p.y = static_cast<Tin*>(d.y);
  p.T = d.T;
  p.H = d.H;
  p.full_batch = d.full_batch;
  p.use_dither = d.use_dither;
  const dim3 grid(d.H, d.Ba, 1), block(kThreads, 1, 1);
  if (d.T == 1)
    hipLaunchKernelGGL((wkv7_infer_kernel<Tin, 1>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((wkv7_infer_kernel<Tin, 16>), grid, block, 0, stream, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_infer(const InferDesc& d, hipStream_t stream) {
  if (d.Ba == 0 || d.H == 0) return hipSuccess;
  return d.dtype == Dtype::BF16 ? launch_infer_t<bf16_t>(d, stream) : launch_infer_t<float>(d, stream);
}

}  // namespace wkv7
