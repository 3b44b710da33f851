// Kernels beside the WKV7 operator in a time mixer, fused per side.
//
// Before the operator -- the token shift and its channel mixes
// (token_shift_diff/kernel.rs:17-64 followed by addcmul5 / addcmul,
// addcmul/kernel.rs:4-53, as WeightPrepare::forward and ChannelMixer::forward
// call them, weight_prepare.rs:221-268, channel_mixer/mod.rs:96-106):
//   prev_t = x_{t-1} if step t-1 is valid, else the external shift (t = 0 too)
//   diff_t = prev_t - x_t (0 at a masked step)
//   mix_i  = x_t + diff_t * scale_i[channel]            for i < num_mixes
// and its backward (token_shift_diff/backward.rs:44-101, addcmul/backward.rs:
// 34-58): with dd_t = sum_i g_i scale_i + g_diff and masked mdd_t = m_t dd_t,
//   dx_t     = sum_i g_i - mdd_t + m_t mdd_{t+1}          (t + 1 < T)
//   dshift_b = sum_t m_t (1 - m_{t-1}) mdd_t               (m_{-1} = 0)
//   dscale_i = sum_{b,t} g_i diff_t
// The difference stays in fp32 between the shift and the mixes.
//
// Before the operator too -- the element-wise end of the weight preparation
// (weight_prepare.rs:282-317), from the projections' and LoRAs' products
// (the LoRA biases added here, layers/lora.rs:118-123):
//   lr  = sigmoid(lr_lora + lr_bias)
//   k~  = key * (key_replacement * (lr - 1) + 1)
//   v   = lerp(value, value_first, sigmoid(vr_lora + vr_bias))   (not cell 0)
//   w   = -softplus(-(wd_lora + wd_bias)) - 0.5
//   u   = rk / max(|rk|_head, 1e-12), rk = key * key_removal
//   a   = -u,  b = u * lr
// and its backward, which recomputes the forward from the same inputs.
//
// After the operator -- the gated readout (gated_readout.rs:110-148):
//   out = (GroupNorm_h(y) + (sum_n r k bonus_h) v) * gate
// with one group per head (64 channels, biased variance, eps), and its
// backward, which recomputes the row statistics instead of storing them.
//
// All of these move a few bytes per flop: they are HBM-bound element-wise
// passes. Each thread owns 4 consecutive channels (one 8- or 16-byte access
// per tensor and row) and walks a short run of rows; the column sums of the
// backward (scale, weight, bias, bonus and the weight preparation's
// per-channel gradients) are reduced within a
// block, written as one partial per block to a workspace and summed in a
// fixed order by a second kernel, so results do not depend on scheduling.
#include <atomic>
#include <mutex>
#include <type_traits>

#include "neighbors_launch.hpp"

namespace rwkv_nb {
namespace {

struct F4 {
  float v[4];
};

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(b) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

template <bool BF>
__device__ __forceinline__ F4 load4(const void* base, int64_t i) {
  F4 o;
  if constexpr (BF) {
    const uint2 raw = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + i);
    o.v[0] = bf16_to_f32(raw.x & 0xffffu);
    o.v[1] = bf16_to_f32(raw.x >> 16);
    o.v[2] = bf16_to_f32(raw.y & 0xffffu);
    o.v[3] = bf16_to_f32(raw.y >> 16);
  } else {
    const float4 f = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + i);
    o.v[0] = f.x;
    o.v[1] = f.y;
    o.v[2] = f.z;
    o.v[3] = f.w;
  }
  return o;
}

template <bool BF>
__device__ __forceinline__ void store4(void* base, int64_t i, const F4& x) {
  if constexpr (BF) {
    uint2 raw;
    raw.x = f32_to_bf16(x.v[0]) | (static_cast<uint32_t>(f32_to_bf16(x.v[1])) << 16);
    raw.y = f32_to_bf16(x.v[2]) | (static_cast<uint32_t>(f32_to_bf16(x.v[3])) << 16);
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(base) + i) = raw;
  } else {
    *reinterpret_cast<float4*>(static_cast<float*>(base) + i) =
        make_float4(x.v[0], x.v[1], x.v[2], x.v[3]);
  }
}

template <bool BF>
__device__ __forceinline__ float load1(const void* base, int64_t i) {
  if constexpr (BF)
    return bf16_to_f32(static_cast<const uint16_t*>(base)[i]);
  else
    return static_cast<const float*>(base)[i];
}

__device__ __forceinline__ F4 zero4() { return F4{{0.f, 0.f, 0.f, 0.f}}; }

// sum over the 16 lanes of a row group
__device__ __forceinline__ float sum16(float x) {
  x += __shfl_xor(x, 8);
  x += __shfl_xor(x, 4);
  x += __shfl_xor(x, 2);
  x += __shfl_xor(x, 1);
  return x;
}

// ------------------------------------------------------------ token shift mix
// slot of row b in the full-batch shift buffers; -1 when a batch id is out
// of range (such a row reads a zero shift and writes no shift or gradient)
__device__ __forceinline__ int64_t slot_of(const ShiftMixArgs& a, int64_t b) {
  const int64_t slot = a.batch_ids ? a.batch_ids[b] : b;
  return (slot >= 0 && slot < a.full_batch) ? slot : -1;
}

template <bool XB>
__device__ __forceinline__ F4 external_shift(const ShiftMixArgs& a, int64_t b, int64_t c) {
  if (!a.shift) return zero4();
  const int64_t slot = slot_of(a, b);
  return slot >= 0 ? load4<XB>(a.shift, slot * a.C + c) : zero4();
}

template <bool XB>
__device__ __forceinline__ bool valid(const ShiftMixArgs& a, int64_t r) {
  return !a.mask || load1<XB>(a.mask, r) != 0.f;
}

// Raw 4-element loads, widened later, so that a group of rows can have all
// its loads in flight before any is used
template <bool BF> struct Raw4;
template <> struct Raw4<true> {
  typedef uint2 type;
  static __device__ __forceinline__ type load(const void* base, int64_t i) {
    return *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + i);
  }
  static __device__ __forceinline__ F4 widen(type r) {
    return F4{{bf16_to_f32(r.x & 0xffffu), bf16_to_f32(r.x >> 16), bf16_to_f32(r.y & 0xffffu),
               bf16_to_f32(r.y >> 16)}};
  }
};
template <> struct Raw4<false> {
  typedef float4 type;
  static __device__ __forceinline__ type load(const void* base, int64_t i) {
    return *reinterpret_cast<const float4*>(static_cast<const float*>(base) + i);
  }
  static __device__ __forceinline__ F4 widen(type r) { return F4{{r.x, r.y, r.z, r.w}}; }
};

// KM: the largest mix count an instantiation serves (1, 6 or 8), so that
// its per-thread arrays hold only as many mixes as the call can have.
//
// A wave's rows, in three phases: every x and mask load of its rows (and of
// the row before them) is issued first, row indices clamped to the tensor so
// that the loads need no branch; then the external shifts, loaded only for
// rows that start a sequence or follow a masked step; then each row's mixes
// are computed and stored. The store phase has no loads, so nothing waits
// for a store: on this hardware a wait for a load also waits for every store
// issued before it. (One row's loads in flight per wave, each behind the
// previous row's stores, left the kernel bound by memory latency.)
template <bool XB, bool OB, int KM>
__global__ __launch_bounds__(256) void shift_mix_forward_kernel(ShiftMixArgs a) {
  constexpr int R = kMixRowsPerWave;
  typedef Raw4<XB> RX;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t C = a.C;
  const int64_t c = (static_cast<int64_t>(blockIdx.y) * 64 + lane) * 4;
  const int64_t rows = a.batch * a.T;
  const int64_t r0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * R;
  const int64_t r1 = r0 + R < rows ? r0 + R : rows;
  if (c >= C || r0 >= r1) return;
  const int n = static_cast<int>(r1 - r0);
  // the scales first: their loads sit under a branch (there may be none), and
  // a wait for them then waits for no row load
  F4 mu[KM];
#pragma unroll
  for (int k = 0; k < KM; ++k)
    mu[k] = k < a.num_mixes ? load4<false>(a.scales, k * C + c) : zero4();
  // the mask, or x standing in for it when there is none (in bounds at every
  // row index, value ignored), so that its loads need no branch either
  const void* const mp = a.mask ? a.mask : a.x;
  // slot 0 is the row before the first (read as row r0 when r0 = 0: unused)
  typename RX::type xr[R + 1];
  float mr[R + 1];
#pragma unroll
  for (int i = 0; i <= R; ++i) {
    const int64_t r = r0 - 1 + (i == 0 ? (r0 > 0 ? 0 : 1) : (i <= n ? i : n));
    xr[i] = RX::load(a.x, r * C + c);
    mr[i] = load1<XB>(mp, r);
  }
  // which rows take the external shift (row-uniform, so wave-uniform)
  const int64_t b0 = r0 / a.T, t0 = r0 - b0 * a.T;
  bool ext[R];
  {
    int64_t t = t0;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      ext[i] = t == 0 || (a.mask && mr[i] == 0.f);   // mr[i] is the previous row's mask
      if (++t == a.T) t = 0;
    }
  }
  F4 es[R];
#pragma unroll
  for (int i = 0; i < R; ++i) es[i] = zero4();
  if (a.shift) {
    int64_t b = b0, t = t0;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (i < n && ext[i]) es[i] = external_shift<XB>(a, b, c);
      if (++t == a.T) {
        t = 0;
        ++b;
      }
    }
    // settle these loads here (no store is outstanding yet), so that the
    // store phase never waits on them: vmcnt(0), other counters untouched
    __builtin_amdgcn_s_waitcnt(0x0F70);
  }
#pragma unroll
  for (int i = 0; i < R; ++i) {
    if (i < n) {
      const int64_t r = r0 + i;
      const F4 xt = RX::widen(xr[i + 1]);
      const bool cur_valid = !a.mask || mr[i + 1] != 0.f;
      const F4 prev = ext[i] ? es[i] : RX::widen(xr[i]);
      F4 d;
#pragma unroll
      for (int j = 0; j < 4; ++j) d.v[j] = cur_valid ? prev.v[j] - xt.v[j] : 0.f;
#pragma unroll
      for (int k = 0; k < KM; ++k) {
        if (k < a.num_mixes) {
          F4 o;
#pragma unroll
          for (int j = 0; j < 4; ++j) o.v[j] = xt.v[j] + d.v[j] * mu[k].v[j];
          store4<OB>(a.mixes[k], r * C + c, o);
        }
      }
      if (a.diff) store4<OB>(a.diff, r * C + c, d);
    }
  }
}

// The one-mix instance walks its rows one at a time instead: there a row is
// mostly its x load (16 bytes per lane against one 8-byte store), and the
// phased walk above measured slower for it (9.4 against 8.7 us per launch in
// the config[4] step, same box), while with six mixes it measured faster
// (17.2 against 22.1 us at config[4]'s shape, same box).
template <bool XB, bool OB, int KM>
__global__ __launch_bounds__(256) void shift_mix_forward_serial_kernel(ShiftMixArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t C = a.C;
  const int64_t c = (static_cast<int64_t>(blockIdx.y) * 64 + lane) * 4;
  const int64_t rows = a.batch * a.T;
  const int64_t r0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * kMixRowsPerWave;
  const int64_t r1 = r0 + kMixRowsPerWave < rows ? r0 + kMixRowsPerWave : rows;
  if (c >= C || r0 >= r1) return;
  F4 mu[KM];
#pragma unroll
  for (int i = 0; i < KM; ++i)
    mu[i] = i < a.num_mixes ? load4<false>(a.scales, i * C + c) : zero4();
  int64_t b = r0 / a.T, t = r0 - b * a.T;
  F4 xprev = zero4();
  bool have_prev = false;
  for (int64_t r = r0; r < r1; ++r) {
    const F4 xt = load4<XB>(a.x, r * C + c);
    const bool cur_valid = valid<XB>(a, r);
    F4 prev;
    if (t > 0 && valid<XB>(a, r - 1))
      prev = have_prev ? xprev : load4<XB>(a.x, (r - 1) * C + c);
    else
      prev = external_shift<XB>(a, b, c);
    F4 d;
#pragma unroll
    for (int j = 0; j < 4; ++j) d.v[j] = cur_valid ? prev.v[j] - xt.v[j] : 0.f;
#pragma unroll
    for (int i = 0; i < KM; ++i) {
      if (i < a.num_mixes) {
        F4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) o.v[j] = xt.v[j] + d.v[j] * mu[i].v[j];
        store4<OB>(a.mixes[i], r * C + c, o);
      }
    }
    if (a.diff) store4<OB>(a.diff, r * C + c, d);
    xprev = xt;
    have_prev = true;
    if (++t == a.T) {
      t = 0;
      ++b;
      have_prev = false;
    }
  }
}

// next_shift[slot(b)] = x at the last valid step of row b, else the external
// shift; a separate launch, so next_shift may be the shift buffer itself
template <bool XB>
__global__ __launch_bounds__(256) void shift_next_kernel(ShiftMixArgs a) {
  const int64_t c = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  const int64_t b = blockIdx.y;
  if (c >= a.C) return;
  int64_t t = a.T - 1;
  if (a.mask)
    while (t >= 0 && load1<XB>(a.mask, b * a.T + t) == 0.f) --t;
  const F4 val = t >= 0 ? load4<XB>(a.x, (b * a.T + t) * a.C + c) : external_shift<XB>(a, b, c);
  const int64_t slot = slot_of(a, b);
  if (slot >= 0) store4<XB>(a.next_shift, slot * a.C + c, val);
}

// dd = sum_i g_i scale_i + g_diff at row r
template <bool OB, int KM>
__device__ __forceinline__ F4 diff_grad_at(const ShiftMixArgs& a, const F4 (&mu)[KM],
                                           int64_t r, int64_t c) {
  F4 dd = a.diff_grad ? load4<OB>(a.diff_grad, r * a.C + c) : zero4();
#pragma unroll
  for (int i = 0; i < KM; ++i) {
    if (i < a.num_mixes) {
      const F4 g = load4<OB>(a.mix_grads[i], r * a.C + c);
#pragma unroll
      for (int j = 0; j < 4; ++j) dd.v[j] += g.v[j] * mu[i].v[j];
    }
  }
  return dd;
}

// The backward of a wave's rows: dx_t = sum_i g_i - m_t dd_t + m_t m_(t+1)
// dd_(t+1), with dd_t = sum_i g_i scale_i (+ the diff gradient), the last
// term only within a sequence. Rows are independent except for that term, so
// the rows go in groups of kGroup whose loads (row indices clamped to the
// tensor, so that they need no branch) are all issued before any is used; a
// row's dx is stored when the next row's masked dd is known. (One row's loads
// in flight per wave left the kernel bound by HBM latency.)
template <bool XB, bool OB, int KM>
__global__ __launch_bounds__(256) void shift_mix_backward_kernel(ShiftMixArgs a) {
  __shared__ float red[4][KM][kMixColsPerBlock];
  constexpr int R = kMixRowsPerWave, kGroup = 4;
  static_assert(R % kGroup == 0, "whole groups of rows");
  typedef Raw4<XB> RX;
  typedef Raw4<OB> RG;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t C = a.C;
  const int64_t c = (static_cast<int64_t>(blockIdx.y) * 64 + lane) * 4;
  const int64_t rows = a.batch * a.T;
  const int64_t r0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * R;
  const int64_t r1 = r0 + R < rows ? r0 + R : rows;
  const bool active = c < C;
  F4 mu[KM], acc[KM];
#pragma unroll
  for (int i = 0; i < KM; ++i) {
    mu[i] = (active && i < a.num_mixes) ? load4<false>(a.scales, i * C + c) : zero4();
    acc[i] = zero4();
  }
  if (active && r0 < r1) {
    const int n = static_cast<int>(r1 - r0);
    const int64_t b0 = r0 / a.T, t0 = r0 - b0 * a.T;
    // the row before the first, for the first row's difference
    F4 xprev = zero4();
    bool prev_valid = false;
    if (t0 > 0) {
      xprev = load4<XB>(a.x, (r0 - 1) * C + c);
      prev_valid = valid<XB>(a, r0 - 1);
    }
    // the previous row, whose dx waits for this row's masked dd
    F4 p_gs = zero4(), p_mdd = zero4();
    float p_m = 0.f;
    int64_t b = b0, t = t0;
    auto store_prev = [&](int i, const F4& next_mdd, bool has_next) {
      F4 dx;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        dx.v[j] = p_gs.v[j] - p_mdd.v[j] + (has_next ? p_m * next_mdd.v[j] : 0.f);
      store4<XB>(a.x_grad, (r0 + i) * C + c, dx);
    };
#pragma unroll
    for (int g0 = 0; g0 < R; g0 += kGroup) {
      typename RX::type xr[kGroup];
      typename RG::type gr[kGroup][KM], dr[kGroup];
      float mr[kGroup];
#pragma unroll
      for (int i = 0; i < kGroup; ++i) {
        const int64_t r = r0 + (g0 + i < n ? g0 + i : n - 1);   // clamped: in bounds, no branch
        xr[i] = RX::load(a.x, r * C + c);
        mr[i] = a.mask ? load1<XB>(a.mask, r) : 1.f;
        if (a.diff_grad) dr[i] = RG::load(a.diff_grad, r * C + c);
#pragma unroll
        for (int k = 0; k < KM; ++k)
          if (k < a.num_mixes) gr[i][k] = RG::load(a.mix_grads[k], r * C + c);
      }
#pragma unroll
      for (int i = 0; i < kGroup; ++i) {
        if (g0 + i < n) {
          const float m = mr[i];
          const F4 xt = RX::widen(xr[i]);
          const F4 prev = (t > 0 && prev_valid) ? xprev : external_shift<XB>(a, b, c);
          F4 d;
#pragma unroll
          for (int j = 0; j < 4; ++j) d.v[j] = m != 0.f ? prev.v[j] - xt.v[j] : 0.f;
          F4 dd = a.diff_grad ? RG::widen(dr[i]) : zero4();
          F4 gs = zero4();
#pragma unroll
          for (int k = 0; k < KM; ++k) {
            if (k < a.num_mixes) {
              const F4 g = RG::widen(gr[i][k]);
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                dd.v[j] += g.v[j] * mu[k].v[j];
                gs.v[j] += g.v[j];
                acc[k].v[j] += g.v[j] * d.v[j];
              }
            }
          }
          F4 mdd;
#pragma unroll
          for (int j = 0; j < 4; ++j) mdd.v[j] = m * dd.v[j];
          // the previous row is in this row's sequence unless this row starts one
          if (g0 + i > 0) store_prev(g0 + i - 1, mdd, t > 0);
          p_gs = gs;
          p_mdd = mdd;
          p_m = m;
          xprev = xt;
          prev_valid = m != 0.f;
          if (++t == a.T) {
            t = 0;
            ++b;
          }
        }
      }
    }
    // the last row: the row after it, when it is in the same sequence (t is
    // now that row's step, 0 when a new sequence starts there)
    F4 after = zero4();
    if (t > 0) {
      const float m = a.mask ? load1<XB>(a.mask, r1) : 1.f;
      const F4 dd = diff_grad_at<OB, KM>(a, mu, r1, c);
#pragma unroll
      for (int j = 0; j < 4; ++j) after.v[j] = m * dd.v[j];
    }
    store_prev(n - 1, after, t > 0);
  }
  // block partial of the scale gradients: the four waves hold the same channels
#pragma unroll
  for (int i = 0; i < KM; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) red[wave][i][lane * 4 + j] = acc[i].v[j];
  __syncthreads();
  if (wave == 0 && active) {
#pragma unroll
    for (int i = 0; i < KM; ++i) {
      if (i < a.num_mixes) {
        F4 s;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          s.v[j] = red[0][i][lane * 4 + j] + red[1][i][lane * 4 + j] +
                   red[2][i][lane * 4 + j] + red[3][i][lane * 4 + j];
        store4<false>(a.workspace, (static_cast<int64_t>(blockIdx.x) * a.num_mixes + i) * C + c, s);
      }
    }
  }
}

// The one-mix instance of the backward, in two phases like the six-mix
// forward: every load is issued first -- the rows' x, masks and gradients,
// the x and mask of the row before them (the first row's difference) and the
// mask and gradients of the row after them (the last row's next-step term),
// row indices clamped to the tensor -- and waited for before the first store;
// then the rows are computed and a row's dx stored once the next row's
// masked dd is known. The store phase loads only an external shift (a row
// that starts a sequence or follows a masked step) and waits for it inside
// that branch. It measured 12.2 against 13.9 us per launch for the grouped
// walk above at config[4]'s shape (same box; bit-identical results). With
// six mixes, holding every row's gradients takes 249 registers, two waves
// per SIMD instead of three, and measured 37.3 against 29.8 us.
template <bool XB, bool OB, int KM>
__global__ __launch_bounds__(256) void shift_mix_backward_phased_kernel(ShiftMixArgs a) {
  __shared__ float red[4][KM][kMixColsPerBlock];
  constexpr int R = kMixRowsPerWave;
  typedef Raw4<XB> RX;
  typedef Raw4<OB> RG;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t C = a.C;
  const int64_t c = (static_cast<int64_t>(blockIdx.y) * 64 + lane) * 4;
  const int64_t rows = a.batch * a.T;
  const int64_t r0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * R;
  const int64_t r1 = r0 + R < rows ? r0 + R : rows;
  const bool active = c < C;
  F4 mu[KM], acc[KM];
#pragma unroll
  for (int i = 0; i < KM; ++i) {
    mu[i] = (active && i < a.num_mixes) ? load4<false>(a.scales, i * C + c) : zero4();
    acc[i] = zero4();
  }
  if (active && r0 < r1) {
    const int n = static_cast<int>(r1 - r0);
    const int64_t b0 = r0 / a.T, t0 = r0 - b0 * a.T;
    auto clamped = [&](int64_t r) { return r < 0 ? int64_t{0} : (r < rows ? r : rows - 1); };
    // the mask, or x standing in for it when there is none (value ignored)
    const void* const mp = a.mask ? a.mask : a.x;
    // slot i of xr / mr: row r0 - 1 + i (slot 0 the row before the first)
    typename RX::type xr[R + 1];
    float mr[R + 1];
#pragma unroll
    for (int i = 0; i <= R; ++i) {
      const int64_t r = clamped(r0 - 1 + (i <= n ? i : n));
      xr[i] = RX::load(a.x, r * C + c);
      mr[i] = load1<XB>(mp, r);
    }
    // slot i of gr / dr: row r0 + i, slot R the row after the last (r1). Past
    // a short run (the tensor's end, so a sequence's end) nothing reads them.
    typename RG::type gr[R + 1][KM], dr[R + 1];
#pragma unroll
    for (int i = 0; i <= R; ++i) {
      const int64_t r = clamped(i < n ? r0 + i : (i == R ? r1 : r1 - 1));
      if (a.diff_grad) dr[i] = RG::load(a.diff_grad, r * C + c);
#pragma unroll
      for (int k = 0; k < KM; ++k)
        if (k < a.num_mixes) gr[i][k] = RG::load(a.mix_grads[k], r * C + c);
    }
    const float m_after = a.mask ? load1<XB>(mp, clamped(r1)) : 1.f;
    // every load has landed before the first store: vmcnt(0), others untouched
    __builtin_amdgcn_s_waitcnt(0x0F70);
    // dd = sum_k g_k scale_k (+ the diff gradient) and gs = sum_k g_k at slot i
    auto grads_at = [&](int i, F4& dd, F4& gs, const F4* d) {
      dd = a.diff_grad ? RG::widen(dr[i]) : zero4();
      gs = zero4();
#pragma unroll
      for (int k = 0; k < KM; ++k) {
        if (k < a.num_mixes) {
          const F4 g = RG::widen(gr[i][k]);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            dd.v[j] += g.v[j] * mu[k].v[j];
            gs.v[j] += g.v[j];
            if (d) acc[k].v[j] += g.v[j] * d->v[j];
          }
        }
      }
    };
    // the previous row, whose dx waits for this row's masked dd
    F4 p_gs = zero4(), p_mdd = zero4();
    float p_m = 0.f;
    auto store_prev = [&](int i, const F4& next_mdd, bool has_next) {
      F4 dx;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        dx.v[j] = p_gs.v[j] - p_mdd.v[j] + (has_next ? p_m * next_mdd.v[j] : 0.f);
      store4<XB>(a.x_grad, (r0 + i) * C + c, dx);
    };
    F4 xprev = RX::widen(xr[0]);
    bool prev_valid = t0 > 0 && (!a.mask || mr[0] != 0.f);
    int64_t b = b0, t = t0;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (i < n) {
        const float m = a.mask ? mr[i + 1] : 1.f;
        const F4 xt = RX::widen(xr[i + 1]);
        F4 prev = xprev;
        if (!(t > 0 && prev_valid)) {
          prev = zero4();
          if (a.shift) {
            prev = external_shift<XB>(a, b, c);
            __builtin_amdgcn_s_waitcnt(0x0F70);   // settled on this path only
          }
        }
        F4 d;
#pragma unroll
        for (int j = 0; j < 4; ++j) d.v[j] = m != 0.f ? prev.v[j] - xt.v[j] : 0.f;
        F4 dd, gs;
        grads_at(i, dd, gs, &d);
        F4 mdd;
#pragma unroll
        for (int j = 0; j < 4; ++j) mdd.v[j] = m * dd.v[j];
        // the previous row is in this row's sequence unless this row starts one
        if (i > 0) store_prev(i - 1, mdd, t > 0);
        p_gs = gs;
        p_mdd = mdd;
        p_m = m;
        xprev = xt;
        prev_valid = m != 0.f;
        if (++t == a.T) {
          t = 0;
          ++b;
        }
      }
    }
    // the last row: the row after it, when it is in the same sequence (t is
    // now that row's step, 0 when a new sequence starts there)
    F4 after = zero4();
    if (t > 0) {
      F4 dd, gs;
      grads_at(R, dd, gs, nullptr);
#pragma unroll
      for (int j = 0; j < 4; ++j) after.v[j] = m_after * dd.v[j];
    }
    store_prev(n - 1, after, t > 0);
  }
  // block partial of the scale gradients: the four waves hold the same channels
#pragma unroll
  for (int i = 0; i < KM; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) red[wave][i][lane * 4 + j] = acc[i].v[j];
  __syncthreads();
  if (wave == 0 && active) {
#pragma unroll
    for (int i = 0; i < KM; ++i) {
      if (i < a.num_mixes) {
        F4 s;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          s.v[j] = red[0][i][lane * 4 + j] + red[1][i][lane * 4 + j] +
                   red[2][i][lane * 4 + j] + red[3][i][lane * 4 + j];
        store4<false>(a.workspace, (static_cast<int64_t>(blockIdx.x) * a.num_mixes + i) * C + c, s);
      }
    }
  }
}

// the external shift's gradient as the reference's autodiff forms it
// (token_shift_diff/backward.rs:51-97): the masked diff gradient m_t dd_t
// weighted by m_t (1 - m_(t-1)) (m_(-1) = 0), summed over the steps, and
// added into the row's slot (select_assign with Add): rows whose batch ids
// repeat add up. The buffer is zero-filled before; with distinct ids each
// slot receives one addition, so the result does not depend on order. For
// 0/1 masks the weight picks the valid steps whose previous step is masked.
template <bool XB, bool OB, int KM>
__global__ __launch_bounds__(256) void shift_grad_kernel(ShiftMixArgs a) {
  const int64_t c = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  const int64_t b = blockIdx.y;
  if (c >= a.C) return;
  F4 mu[KM];
#pragma unroll
  for (int i = 0; i < KM; ++i)
    mu[i] = i < a.num_mixes ? load4<false>(a.scales, i * a.C + c) : zero4();
  F4 acc = zero4();
  float mprev = 0.f;
  for (int64_t t = 0; t < a.T; ++t) {
    const int64_t r = b * a.T + t;
    const float m = a.mask ? load1<XB>(a.mask, r) : 1.f;
    const float w = m * (1.f - mprev);   // use_external_shift
    if (w != 0.f) {
      const F4 dd = diff_grad_at<OB, KM>(a, mu, r, c);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc.v[j] += (dd.v[j] * m) * w;
    }
    mprev = m;
    if (!a.mask) break;  // without a mask only t = 0 has a weight
  }
  const int64_t slot = slot_of(a, b);
  if (slot >= 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) atomicAdd(a.shift_grad + slot * a.C + c + j, acc.v[j]);
  }
}

__global__ __launch_bounds__(256) void fill_zero_kernel(float* p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

// out_q[c] = sum over row blocks of ws[rb][q][c]: 16 waves split the row
// blocks (wave w takes w, w + 16, ...), each sums its share in order, then
// the 16 partial sums are added in wave order, so the result is the same on
// every run
constexpr int kSumWaves = 16;

struct ColumnSumArgs {
  const float* ws;
  int64_t row_blocks, Q, C;
  float* out[kMaxMixes];
};

__global__ __launch_bounds__(64 * kSumWaves) void column_sum_kernel(ColumnSumArgs a) {
  __shared__ float red[kSumWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 64 + lane;
  const int q = blockIdx.y;
  // kBatch partials in flight per wave (indices clamped, so the loads need no
  // branch), added in the same order as one at a time
  constexpr int kBatch = 8;
  float s = 0.f;
  if (c < a.C)
    for (int64_t rb0 = wave; rb0 < a.row_blocks; rb0 += kSumWaves * kBatch) {
      float x[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int64_t rb = rb0 + i * kSumWaves;
        x[i] = a.ws[((rb < a.row_blocks ? rb : a.row_blocks - 1) * a.Q + q) * a.C + c];
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i)
        if (rb0 + i * kSumWaves < a.row_blocks) s += x[i];
    }
  red[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && c < a.C) {
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < kSumWaves; ++w) tot += red[w][lane];
#pragma unroll
    for (int i = 0; i < kMaxMixes; ++i)
      if (i == q) a.out[i][c] = tot;
  }
}

// -------------------------------------------------------------- gated readout
// A row's group-norm statistics and bonus term: yh = (y - mean) rstd over the
// head's 64 channels, s = sum_n r k bonus (16 lanes of 4 channels).
__device__ __forceinline__ void readout_stats(float eps, const F4& rk, const F4& y, const F4& r,
                                              const F4& k, F4& yh, float& rstd, float& s) {
  const float mean = sum16(y.v[0] + y.v[1] + y.v[2] + y.v[3]) * (1.f / 64.f);
  float d2 = 0.f, bon = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    yh.v[j] = y.v[j] - mean;
    d2 += yh.v[j] * yh.v[j];
    bon += r.v[j] * k.v[j] * rk.v[j];
  }
  rstd = rsqrtf(sum16(d2) * (1.f / 64.f) + eps);
#pragma unroll
  for (int j = 0; j < 4; ++j) yh.v[j] *= rstd;
  s = sum16(bon);
}

// Both readout kernels: a 16-lane group walks kReadoutRowsPerGroup rows of
// one head. All of the group's loads are issued before any row is used (row
// indices clamped to the tensor, so the loads need no branch); rows past the
// end are computed on the clamped data and not stored. (One row's loads in
// flight per group left these kernels bound by HBM latency.)
template <bool OPB, bool ACTB>
__global__ __launch_bounds__(256) void readout_forward_kernel(ReadoutArgs a) {
  constexpr int R = kReadoutRowsPerGroup;
  typedef Raw4<OPB> RO;
  typedef Raw4<ACTB> RA;
  const int grp = threadIdx.x >> 4, l = threadIdx.x & 15;
  const int64_t C = a.H * 64;
  const int64_t cc = static_cast<int64_t>(blockIdx.y) * 64 + l * 4;
  const int64_t r0 = (static_cast<int64_t>(blockIdx.x) * 16 + grp) * R;
  if (r0 >= a.rows) return;  // uniform over the group; no block-wide sync follows
  const int n = a.rows - r0 < R ? static_cast<int>(a.rows - r0) : R;
  typename RO::type yr[R], rr[R], kr[R], vr[R];
  typename RA::type gr[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int64_t idx = (r0 + (i < n ? i : n - 1)) * C + cc;
    yr[i] = RO::load(a.y, idx);
    rr[i] = RO::load(a.r, idx);
    kr[i] = RO::load(a.k, idx);
    vr[i] = RO::load(a.v, idx);
    gr[i] = RA::load(a.gate, idx);
  }
  const F4 gw = load4<false>(a.weight, cc), gb = load4<false>(a.bias, cc);
  const F4 rk = load4<false>(a.bonus, cc);
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const F4 v = RO::widen(vr[i]), g = RA::widen(gr[i]);
    F4 yh;
    float rstd, s;
    readout_stats(a.eps, rk, RO::widen(yr[i]), RO::widen(rr[i]), RO::widen(kr[i]), yh, rstd, s);
    F4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o.v[j] = (yh.v[j] * gw.v[j] + gb.v[j] + s * v.v[j]) * g.v[j];
    if (i < n) store4<ACTB>(a.out, (r0 + i) * C + cc, o);
  }
}

template <bool OPB, bool ACTB>
__global__ __launch_bounds__(256) void readout_backward_kernel(ReadoutArgs a) {
  constexpr int R = kReadoutRowsPerGroup;
  typedef Raw4<OPB> RO;
  typedef Raw4<ACTB> RA;
  __shared__ float red[16][kReadoutSums][64];
  const int grp = threadIdx.x >> 4, l = threadIdx.x & 15;
  const int64_t C = a.H * 64;
  const int64_t cc = static_cast<int64_t>(blockIdx.y) * 64 + l * 4;
  F4 aw = zero4(), ab = zero4(), ak = zero4();
  const int64_t r0 = (static_cast<int64_t>(blockIdx.x) * 16 + grp) * R;
  if (r0 < a.rows) {  // uniform over the group
    const int n = a.rows - r0 < R ? static_cast<int>(a.rows - r0) : R;
    typename RO::type yr[R], rr[R], kr[R], vr[R];
    typename RA::type gr[R], dr[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int64_t idx = (r0 + (i < n ? i : n - 1)) * C + cc;
      yr[i] = RO::load(a.y, idx);
      rr[i] = RO::load(a.r, idx);
      kr[i] = RO::load(a.k, idx);
      vr[i] = RO::load(a.v, idx);
      gr[i] = RA::load(a.gate, idx);
      dr[i] = RA::load(a.out_grad, idx);
    }
    const F4 gw = load4<false>(a.weight, cc), gb = load4<false>(a.bias, cc);
    const F4 rk = load4<false>(a.bonus, cc);
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const F4 r = RO::widen(rr[i]), k = RO::widen(kr[i]), v = RO::widen(vr[i]);
      const F4 g = RA::widen(gr[i]), dout = RA::widen(dr[i]);
      F4 yh;
      float rstd, s;
      readout_stats(a.eps, rk, RO::widen(yr[i]), r, k, yh, rstd, s);
      const bool live = i < n;  // a row past the end adds nothing to the column sums
      F4 dz, dg, dv, dyh;
      float ds = 0.f, m1 = 0.f, m2 = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float z = yh.v[j] * gw.v[j] + gb.v[j] + s * v.v[j];
        dz.v[j] = dout.v[j] * g.v[j];
        dg.v[j] = dout.v[j] * z;
        aw.v[j] = live ? aw.v[j] + dz.v[j] * yh.v[j] : aw.v[j];
        ab.v[j] = live ? ab.v[j] + dz.v[j] : ab.v[j];
        dv.v[j] = dz.v[j] * s;
        ds += dz.v[j] * v.v[j];
        dyh.v[j] = dz.v[j] * gw.v[j];
        m1 += dyh.v[j];
        m2 += dyh.v[j] * yh.v[j];
      }
      ds = sum16(ds);
      m1 = sum16(m1) * (1.f / 64.f);
      m2 = sum16(m2) * (1.f / 64.f);
      F4 drr, dk, dy;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        drr.v[j] = ds * k.v[j] * rk.v[j];
        dk.v[j] = ds * r.v[j] * rk.v[j];
        ak.v[j] = live ? ak.v[j] + ds * r.v[j] * k.v[j] : ak.v[j];
        dy.v[j] = rstd * (dyh.v[j] - m1 - yh.v[j] * m2);
      }
      if (live) {
        const int64_t idx = (r0 + i) * C + cc;
        store4<ACTB>(a.gate_grad, idx, dg);
        store4<OPB>(a.v_grad, idx, dv);
        store4<OPB>(a.r_grad, idx, drr);
        store4<OPB>(a.k_grad, idx, dk);
        store4<OPB>(a.y_grad, idx, dy);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    red[grp][0][l * 4 + j] = aw.v[j];
    red[grp][1][l * 4 + j] = ab.v[j];
    red[grp][2][l * 4 + j] = ak.v[j];
  }
  __syncthreads();
  if (threadIdx.x < kReadoutSums * 64) {
    const int q = threadIdx.x >> 6, n = threadIdx.x & 63;
    float s = 0.f;
    for (int g = 0; g < 16; ++g) s += red[g][q][n];
    a.workspace[(static_cast<int64_t>(blockIdx.x) * kReadoutSums + q) * C +
                static_cast<int64_t>(blockIdx.y) * 64 + n] = s;
  }
}

// ------------------------------------------------- weight preparation, end
constexpr float kNormEps = 1e-12f;       // F.normalize's eps (weight_prepare.rs:313)
constexpr float kSoftplusLinear = 20.f;  // softplus(y) = y above this, as torch's

__device__ __forceinline__ float sigmoid1(float x) { return 1.f / (1.f + expf(-x)); }

__device__ __forceinline__ float softplus1(float y) {
  return y > kSoftplusLinear ? y : log1pf(expf(y));
}

// softplus'(y)
__device__ __forceinline__ float softplus_slope(float y) {
  return y > kSoftplusLinear ? 1.f : sigmoid1(y);
}

// the forward of one row's four channels, kept for the backward
struct PrepareRow {
  F4 k;       // key precursor
  F4 lr;      // learning rate
  F4 alpha;   // key_replacement * (lr - 1) + 1
  F4 wd;      // decay LoRA output with its bias
  F4 u;       // normalized removal key (before the sign)
  F4 v;       // value after the residual
  F4 nu;      // value-residual gate (RES)
  F4 vdiff;   // value_first - value (RES)
  float den;  // max(|rk|, eps) of the row's head
  bool clamped;
};

struct PrepareParams {
  F4 lr_bias, wd_bias, vr_bias, ka, kk;
};

template <bool RES>
__device__ __forceinline__ PrepareParams prepare_params(const PrepareArgs& a, int64_t cc) {
  PrepareParams q;
  q.lr_bias = load4<false>(a.lr_bias, cc);
  q.wd_bias = load4<false>(a.wd_bias, cc);
  q.vr_bias = RES ? load4<false>(a.vr_bias, cc) : zero4();
  q.ka = load4<false>(a.key_replacement, cc);
  q.kk = load4<false>(a.key_removal, cc);
  return q;
}

template <bool IB, bool RES>
__device__ __forceinline__ void prepare_row(const PrepareArgs& a, int64_t idx,
                                            const PrepareParams& q, PrepareRow& p) {
  p.k = load4<IB>(a.key, idx);
  const F4 lr = load4<IB>(a.lr, idx), wd = load4<IB>(a.wd, idx), vp = load4<IB>(a.value, idx);
  F4 vf = zero4(), vr = zero4();
  if constexpr (RES) {
    vf = load4<IB>(a.value_first, idx);
    vr = load4<IB>(a.vr, idx);
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    p.lr.v[j] = sigmoid1(lr.v[j] + q.lr_bias.v[j]);
    p.alpha.v[j] = q.ka.v[j] * (p.lr.v[j] - 1.f) + 1.f;
    p.wd.v[j] = wd.v[j] + q.wd_bias.v[j];
    p.u.v[j] = p.k.v[j] * q.kk.v[j];
    ss += p.u.v[j] * p.u.v[j];
    if constexpr (RES) {
      p.nu.v[j] = sigmoid1(vr.v[j] + q.vr_bias.v[j]);
      p.vdiff.v[j] = vf.v[j] - vp.v[j];
      p.v.v[j] = vp.v[j] + p.vdiff.v[j] * p.nu.v[j];
    } else {
      p.v.v[j] = vp.v[j];
    }
  }
  const float n = sqrtf(sum16(ss));
  p.clamped = !(n >= kNormEps);  // x / clamp_min(|x|, eps); no gradient through a clamped norm
  p.den = p.clamped ? kNormEps : n;
#pragma unroll
  for (int j = 0; j < 4; ++j) p.u.v[j] = p.u.v[j] / p.den;
}

template <bool IB, bool OB, bool RES>
__global__ __launch_bounds__(256) void prepare_forward_kernel(PrepareArgs a) {
  const int grp = threadIdx.x >> 4, l = threadIdx.x & 15;
  const int64_t C = a.H * 64;
  const int64_t cc = static_cast<int64_t>(blockIdx.y) * 64 + l * 4;
  const PrepareParams q = prepare_params<RES>(a, cc);
  const int64_t r0 = (static_cast<int64_t>(blockIdx.x) * 16 + grp) * kPrepareRowsPerGroup;
  for (int i = 0; i < kPrepareRowsPerGroup; ++i) {
    const int64_t row = r0 + i;
    if (row >= a.rows) break;  // uniform over the 16 lanes of the group
    const int64_t idx = row * C + cc;
    PrepareRow p;
    prepare_row<IB, RES>(a, idx, q, p);
    F4 w, kt, na, b;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      w.v[j] = -softplus1(-p.wd.v[j]) - 0.5f;
      kt.v[j] = p.k.v[j] * p.alpha.v[j];
      na.v[j] = -p.u.v[j];
      b.v[j] = p.u.v[j] * p.lr.v[j];
    }
    store4<OB>(a.weight_decay, idx, w);
    store4<OB>(a.replacement_key, idx, kt);
    store4<OB>(a.value_out, idx, p.v);
    store4<OB>(a.removal, idx, na);
    store4<OB>(a.replacement, idx, b);
  }
}

template <bool IB, bool OB, bool RES>
__global__ __launch_bounds__(256) void prepare_backward_kernel(PrepareArgs a) {
  constexpr int Q = RES ? kPrepareSums : kPrepareSums - 1;
  __shared__ float red[16][kPrepareSums][64];
  const int grp = threadIdx.x >> 4, l = threadIdx.x & 15;
  const int64_t C = a.H * 64;
  const int64_t cc = static_cast<int64_t>(blockIdx.y) * 64 + l * 4;
  const PrepareParams q = prepare_params<RES>(a, cc);
  F4 acc[kPrepareSums];
#pragma unroll
  for (int s = 0; s < kPrepareSums; ++s) acc[s] = zero4();
  const int64_t r0 = (static_cast<int64_t>(blockIdx.x) * 16 + grp) * kPrepareRowsPerGroup;
  for (int i = 0; i < kPrepareRowsPerGroup; ++i) {
    const int64_t row = r0 + i;
    if (row >= a.rows) break;  // uniform over the 16 lanes of the group
    const int64_t idx = row * C + cc;
    PrepareRow p;
    prepare_row<IB, RES>(a, idx, q, p);
    const F4 gw = load4<OB>(a.weight_decay_grad, idx), gkt = load4<OB>(a.replacement_key_grad, idx);
    const F4 gv = load4<OB>(a.value_out_grad, idx), ga = load4<OB>(a.removal_grad, idx);
    const F4 gb = load4<OB>(a.replacement_grad, idx);
    // a = -u and b = u lr: the gradient reaching u, and u . du over the head
    F4 du;
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      du.v[j] = gb.v[j] * p.lr.v[j] - ga.v[j];
      dot += p.u.v[j] * du.v[j];
    }
    dot = sum16(dot);
    F4 dk, dlr, dwd, dvp, dvf, dvr;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // u = rk / den: d rk = (du - u (u . du)) / |rk|, or du / eps when clamped
      const float drk = p.clamped ? du.v[j] / kNormEps : (du.v[j] - p.u.v[j] * dot) / p.den;
      const float dalpha = gkt.v[j] * p.k.v[j];
      const float glr = gb.v[j] * p.u.v[j] + dalpha * q.ka.v[j];
      dlr.v[j] = glr * p.lr.v[j] * (1.f - p.lr.v[j]);
      dk.v[j] = gkt.v[j] * p.alpha.v[j] + drk * q.kk.v[j];
      dwd.v[j] = gw.v[j] * softplus_slope(-p.wd.v[j]);
      acc[PS_LR_BIAS].v[j] += dlr.v[j];
      acc[PS_WD_BIAS].v[j] += dwd.v[j];
      acc[PS_KEY_REPLACEMENT].v[j] += dalpha * (p.lr.v[j] - 1.f);
      acc[PS_KEY_REMOVAL].v[j] += drk * p.k.v[j];
      if constexpr (RES) {
        const float nu = p.nu.v[j];
        dvp.v[j] = gv.v[j] * (1.f - nu);
        dvf.v[j] = gv.v[j] * nu;
        dvr.v[j] = gv.v[j] * p.vdiff.v[j] * nu * (1.f - nu);
        acc[PS_VR_BIAS].v[j] += dvr.v[j];
      } else {
        dvp.v[j] = gv.v[j];
      }
    }
    store4<IB>(a.key_grad, idx, dk);
    store4<IB>(a.value_grad, idx, dvp);
    store4<IB>(a.lr_grad, idx, dlr);
    store4<IB>(a.wd_grad, idx, dwd);
    if constexpr (RES) {
      store4<IB>(a.value_first_grad, idx, dvf);
      store4<IB>(a.vr_grad, idx, dvr);
    }
  }
#pragma unroll
  for (int s = 0; s < Q; ++s)
#pragma unroll
    for (int j = 0; j < 4; ++j) red[grp][s][l * 4 + j] = acc[s].v[j];
  __syncthreads();
  // Q * 64 partials over the block's 256 threads
  for (int e = threadIdx.x; e < Q * 64; e += 256) {
    const int s = e >> 6, n = e & 63;
    float t = 0.f;
    for (int g = 0; g < 16; ++g) t += red[g][s][n];
    a.workspace[(static_cast<int64_t>(blockIdx.x) * Q + s) * C +
                static_cast<int64_t>(blockIdx.y) * 64 + n] = t;
  }
}

template <typename K>
hipError_t launch(K kernel, dim3 grid, dim3 block, hipStream_t s) {
  hipLaunchKernelGGL(kernel, grid, block, 0, s);
  return hipGetLastError();
}

template <typename K, typename A>
hipError_t launch(K kernel, dim3 grid, dim3 block, hipStream_t s, const A& args) {
  hipLaunchKernelGGL(kernel, grid, block, 0, s, args);
  return hipGetLastError();
}

hipError_t column_sum(const float* ws, int64_t row_blocks, int64_t Q, int64_t C,
                      float* const* outs, hipStream_t s) {
  ColumnSumArgs c{};
  c.ws = ws;
  c.row_blocks = row_blocks;
  c.Q = Q;
  c.C = C;
  for (int i = 0; i < Q; ++i) c.out[i] = outs[i];
  const dim3 grid(static_cast<unsigned>((C + 63) / 64), static_cast<unsigned>(Q));
  return launch(column_sum_kernel, grid, dim3(64 * kSumWaves), s, c);
}

hipError_t fill_zero(float* p, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(fill_zero_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256),
                     0, s, p, n);
  return hipGetLastError();
}

}  // namespace

namespace {

// one instantiation per (x dtype, output dtype, mix-count class)
template <template <bool, bool, int> class Kern>
hipError_t dispatch(const ShiftMixArgs& a, dim3 grid, dim3 block, hipStream_t s) {
  const int km = a.num_mixes <= 1 ? 1 : a.num_mixes <= 6 ? 6 : 8;
  auto go = [&](auto xb, auto ob) -> hipError_t {
    constexpr bool XB = decltype(xb)::value, OB = decltype(ob)::value;
    if (km == 1) return launch(Kern<XB, OB, 1>::fn, grid, block, s, a);
    if (km == 6) return launch(Kern<XB, OB, 6>::fn, grid, block, s, a);
    return launch(Kern<XB, OB, 8>::fn, grid, block, s, a);
  };
  using T = std::true_type;
  using F = std::false_type;
  if (a.x_bf16) return a.out_bf16 ? go(T{}, T{}) : go(T{}, F{});
  return a.out_bf16 ? go(F{}, T{}) : go(F{}, F{});
}

template <bool XB, bool OB, int KM>
struct MixForward {
  static constexpr auto fn = shift_mix_forward_kernel<XB, OB, KM>;
};
template <bool XB, bool OB>
struct MixForward<XB, OB, 1> {
  static constexpr auto fn = shift_mix_forward_serial_kernel<XB, OB, 1>;
};
template <bool XB, bool OB, int KM>
struct MixBackward {
  static constexpr auto fn = shift_mix_backward_kernel<XB, OB, KM>;
};
template <bool XB, bool OB>
struct MixBackward<XB, OB, 1> {
  static constexpr auto fn = shift_mix_backward_phased_kernel<XB, OB, 1>;
};
template <bool XB, bool OB, int KM>
struct ShiftGrad {
  static constexpr auto fn = shift_grad_kernel<XB, OB, KM>;
};

}  // namespace

hipError_t launch_shift_mix_forward(const ShiftMixArgs& a, hipStream_t s) {
  const int64_t rows = a.batch * a.T;
  const unsigned gx = static_cast<unsigned>((a.C + kMixColsPerBlock - 1) / kMixColsPerBlock);
  if (rows > 0) {
    const dim3 grid(static_cast<unsigned>(mix_row_blocks(rows)), gx);
    const hipError_t e = dispatch<MixForward>(a, grid, dim3(256), s);
    if (e != hipSuccess) return e;
  }
  if (a.next_shift && a.batch > 0) {
    const dim3 grid(gx, static_cast<unsigned>(a.batch));
    return a.x_bf16 ? launch(shift_next_kernel<true>, grid, dim3(64), s, a)
                    : launch(shift_next_kernel<false>, grid, dim3(64), s, a);
  }
  return hipSuccess;
}

hipError_t launch_shift_mix_backward(const ShiftMixArgs& a, hipStream_t s) {
  const int64_t rows = a.batch * a.T;
  const unsigned gx = static_cast<unsigned>((a.C + kMixColsPerBlock - 1) / kMixColsPerBlock);
  hipError_t e = hipSuccess;
  if (rows > 0) {
    const int64_t rb = mix_row_blocks(rows);
    e = dispatch<MixBackward>(a, dim3(static_cast<unsigned>(rb), gx), dim3(256), s);
    if (e != hipSuccess) return e;
    if (a.num_mixes > 0) {
      float* outs[kMaxMixes];
      for (int i = 0; i < a.num_mixes; ++i) outs[i] = a.scales_grad + i * a.C;
      e = column_sum(a.workspace, rb, a.num_mixes, a.C, outs, s);
      if (e != hipSuccess) return e;
    }
  } else if (a.num_mixes > 0) {
    e = fill_zero(a.scales_grad, a.num_mixes * a.C, s);
    if (e != hipSuccess) return e;
  }
  if (a.shift_grad) {
    e = fill_zero(a.shift_grad, a.full_batch * a.C, s);
    if (e != hipSuccess) return e;
    if (rows > 0)
      e = dispatch<ShiftGrad>(a, dim3(gx, static_cast<unsigned>(a.batch)), dim3(64), s);
  }
  return e;
}

hipError_t launch_readout_forward(const ReadoutArgs& a, hipStream_t s) {
  if (a.rows == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(readout_row_blocks(a.rows)), static_cast<unsigned>(a.H));
  if (a.op_bf16)
    return a.act_bf16 ? launch(readout_forward_kernel<true, true>, grid, dim3(256), s, a)
                      : launch(readout_forward_kernel<true, false>, grid, dim3(256), s, a);
  return a.act_bf16 ? launch(readout_forward_kernel<false, true>, grid, dim3(256), s, a)
                    : launch(readout_forward_kernel<false, false>, grid, dim3(256), s, a);
}

hipError_t launch_readout_backward(const ReadoutArgs& a, hipStream_t s) {
  const int64_t C = a.H * 64;
  float* outs[kReadoutSums] = {a.weight_grad, a.bias_grad, a.bonus_grad};
  if (a.rows == 0) {
    for (float* p : outs) {
      const hipError_t e = fill_zero(p, C, s);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  const int64_t rb = readout_row_blocks(a.rows);
  const dim3 grid(static_cast<unsigned>(rb), static_cast<unsigned>(a.H));
  hipError_t e;
  if (a.op_bf16)
    e = a.act_bf16 ? launch(readout_backward_kernel<true, true>, grid, dim3(256), s, a)
                   : launch(readout_backward_kernel<true, false>, grid, dim3(256), s, a);
  else
    e = a.act_bf16 ? launch(readout_backward_kernel<false, true>, grid, dim3(256), s, a)
                   : launch(readout_backward_kernel<false, false>, grid, dim3(256), s, a);
  if (e != hipSuccess) return e;
  return column_sum(a.workspace, rb, kReadoutSums, C, outs, s);
}

namespace {

// one instantiation per (input dtype, output dtype, residual or not)
template <template <bool, bool, bool> class Kern>
hipError_t dispatch_prepare(const PrepareArgs& a, dim3 grid, hipStream_t s) {
  auto go = [&](auto ib, auto ob) -> hipError_t {
    constexpr bool IB = decltype(ib)::value, OB = decltype(ob)::value;
    return a.residual ? launch(Kern<IB, OB, true>::fn, grid, dim3(256), s, a)
                         : launch(Kern<IB, OB, false>::fn, grid, dim3(256), s, a);
  };
  using T = std::true_type;
  using F = std::false_type;
  if (a.in_bf16) return a.out_bf16 ? go(T{}, T{}) : go(T{}, F{});
  return a.out_bf16 ? go(F{}, T{}) : go(F{}, F{});
}

template <bool IB, bool OB, bool RES>
struct PrepareForward {
  static constexpr auto fn = prepare_forward_kernel<IB, OB, RES>;
};
template <bool IB, bool OB, bool RES>
struct PrepareBackward {
  static constexpr auto fn = prepare_backward_kernel<IB, OB, RES>;
};

}  // namespace

hipError_t launch_prepare_forward(const PrepareArgs& a, hipStream_t s) {
  if (a.rows == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(prepare_row_blocks(a.rows)), static_cast<unsigned>(a.H));
  return dispatch_prepare<PrepareForward>(a, grid, s);
}

hipError_t launch_prepare_backward(const PrepareArgs& a, hipStream_t s) {
  const int64_t C = a.H * 64;
  const int q = a.residual ? kPrepareSums : kPrepareSums - 1;
  if (a.rows == 0) {
    for (int i = 0; i < q; ++i) {
      const hipError_t e = fill_zero(a.sums[i], C, s);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  const int64_t rb = prepare_row_blocks(a.rows);
  const hipError_t e =
      dispatch_prepare<PrepareBackward>(a, dim3(static_cast<unsigned>(rb), static_cast<unsigned>(a.H)), s);
  if (e != hipSuccess) return e;
  return column_sum(a.workspace, rb, q, C, a.sums, s);
}

// ------------------------------------------------- fixed device scratch array
// The gated readout backward's column-sum partials for callers that cannot
// allocate (rwkv_gated_readout_backward_noalloc). Each GPU holds its own copy
// of `scratch` at its own address for the life of the process. In host code
// the name `scratch` is only a host-side stand-in, so it is never passed to a
// kernel: the device address is looked up once per device with
// hipGetSymbolAddress and kept in scratch_ptr[device] for the life of the
// process. A hipDeviceReset would leave that address stale, so the noalloc
// entry point is not for processes that reset a device they called it on.
namespace {

static __device__ __align__(256) float scratch[kReadoutScratchBytes / sizeof(float)];

constexpr int kMaxScratchDevices = 256;
std::atomic<float*> scratch_ptr[kMaxScratchDevices];
std::mutex scratch_mu;

}  // namespace

hipError_t readout_scratch(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxScratchDevices) return hipErrorInvalidDevice;
  float* p = scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(scratch_mu);
    p = scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      void* addr = nullptr;
      e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return e;
      if (!addr) return hipErrorInvalidSymbol;
      p = static_cast<float*>(addr);
      scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return hipSuccess;
}

}  // namespace rwkv_nb
