// Device-side building blocks shared by the WKV7 kernels (gfx950 / CDNA4).
//
// Work layout. One workgroup (512 threads, 8 waves) owns one (batch, head)
// pair and its 64x64 fp32 state S (row j = value index, column i = key index).
//
// Why eight waves per head: on gfx950 a wave issues at most one VALU
// instruction about every 4 cycles, while a SIMD retires a plain wave64 FP32
// FMA every ~2 cycles when two waves feed it; DPP-modified instructions retire
// at half that rate. With 256 heads (the benchmark shape) only 512 threads per
// head give every SIMD two waves.
//
// Thread tile. Thread tid owns a 2x4 block: column group L = tid % 16
// (columns 4L .. 4L+3) and row pair q = tid / 16 (rows 2q, 2q+1). The sixteen
// lanes of one DPP row therefore cover all 64 columns of two rows, so a sum
// over a row is 4 in-lane products plus a 4-step DPP rotation reduction, and
// every per-column operand the thread needs is one ds_read_b128 of a 64-entry
// LDS vector (entries 4L .. 4L+3), consumed by plain full-rate FMAs.
// LDS bandwidth (~250 B/clk/CU on gfx950, broadcast or not) is the other
// limit, which is why the block is 2x4 rather than 1x8.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wkv7 {

constexpr int kHead = 64;        // head size N (the kernels are specialised)
constexpr int kThreads = 512;    // 8 waves per (batch, head)
constexpr float kWScale = -0.6065306597f;   // -exp(-1/2), kernel.rs:4

typedef uint16_t bf16_t;

// ---------------------------------------------------------------- conversions
__device__ __forceinline__ float bf16_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

// round-to-nearest-even f32 -> bf16 bits (NaN kept quiet)
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// 4 consecutive elements of an fp32 or bf16 tensor: load, widen, store
template <typename T> struct Io;

template <> struct Io<float> {
  typedef float4 raw;
  static __device__ __forceinline__ raw load(const float* p) {
    return *reinterpret_cast<const float4*>(p);
  }
  static __device__ __forceinline__ float4 widen(raw x) { return x; }
  static __device__ __forceinline__ void store(float* p, float4 x) {
    *reinterpret_cast<float4*>(p) = x;
  }
};

template <> struct Io<bf16_t> {
  typedef uint2 raw;
  static __device__ __forceinline__ raw load(const bf16_t* p) {
    return *reinterpret_cast<const uint2*>(p);
  }
  static __device__ __forceinline__ float4 widen(raw x) {
    return make_float4(__uint_as_float(x.x << 16), __uint_as_float(x.x & 0xffff0000u),
                       __uint_as_float(x.y << 16), __uint_as_float(x.y & 0xffff0000u));
  }
  static __device__ __forceinline__ void store(bf16_t* p, float4 x) {
    uint2 o;
    o.x = f32_to_bf16(x.x) | (f32_to_bf16(x.y) << 16);
    o.y = f32_to_bf16(x.z) | (f32_to_bf16(x.w) << 16);
    *reinterpret_cast<uint2*>(p) = o;
  }
};

// decay w~ = exp(W_SCALE * sigmoid(x)), kernel.rs:63-65; also sigmoid(x)
__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float decay_f(float sig) { return expf(kWScale * sig); }

// ------------------------------------------------------- cross-lane reduction
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}

// Sum within each 8-lane half of a DPP row (pairs L/7-L, then L/L^2, then
// L/L^1). All eight lanes get the same bits: every step adds two partial sums
// that the lanes of the orbit form from the same operands, and IEEE addition
// is commutative.
__device__ __forceinline__ float half8_sum(float x) {
  x += dpp_mov<0x141>(x);   // row_half_mirror
  x += dpp_mov<0x4E>(x);    // quad_perm:[2,3,0,1]
  x += dpp_mov<0xB1>(x);    // quad_perm:[1,0,3,2]
  return x;
}

// One recursive-halving step of a reduce-scatter over a DPP row: the lane
// keeps half of its N values (the upper half when `upper`) and adds the
// partner's copy of that half; the partner lane (the DPP source) has the
// opposite `upper`.
template <int CTRL, int N>
__device__ __forceinline__ void rs_step(float* x, bool upper) {
#pragma unroll
  for (int j = 0; j < N / 2; ++j) {
    const float keep = upper ? x[N / 2 + j] : x[j];
    const float send = upper ? x[j] : x[N / 2 + j];
    x[j] = keep + dpp_mov<CTRL>(send);
  }
}

// Sums of N values (N = 2, 4, 8, 16) over the 16 lanes of a DPP row, spread
// over the lanes: afterwards x[0] of lane L holds the full sum of value
// index L / (16/N), i.e. lanes (16/N)*m .. (16/N)*m + 16/N - 1 hold value m. Partners: L^8 (row_ror:8), the mirror inside an 8-lane half, L^2,
// L^1; a level with one value left is a plain pairwise sum.
template <int N>
__device__ __forceinline__ void row16_scatter(float* x, int L) {
  static_assert(N == 2 || N == 4 || N == 8 || N == 16, "N must be 2, 4, 8 or 16");
  rs_step<0x128, N>(x, (L & 8) != 0);
  if constexpr (N >= 4) rs_step<0x141, N / 2>(x, (L & 4) != 0);
  else x[0] += dpp_mov<0x141>(x[0]);
  if constexpr (N >= 8) rs_step<0x4E, N / 4>(x, (L & 2) != 0);
  else x[0] += dpp_mov<0x4E>(x[0]);
  if constexpr (N >= 16) rs_step<0xB1, N / 8>(x, (L & 1) != 0);
  else x[0] += dpp_mov<0xB1>(x[0]);
}

// Both row sums of a lane pair (x0, x1), available in every lane of the DPP
// row: a reduce-scatter to one value per half, then one exchange.
__device__ __forceinline__ void row16_sum2(float& x0, float& x1, int L) {
  float x[2] = {x0, x1};
  row16_scatter<2>(x, L);   // lanes 0-7: sum of x0, lanes 8-15: sum of x1
  const float other = dpp_mov<0x128>(x[0]);
  const bool up = (L & 8) != 0;
  x0 = up ? other : x[0];
  x1 = up ? x[0] : other;
}

// ---------------------------------------------------------- direct LDS loads
// 16 bytes from global memory to LDS without passing through VGPRs
// (global_load_lds_dwordx4, new in gfx950). `lds_wave_base` must be the same
// for the whole wave: lane i writes lds_wave_base + 16 * i. Completion is
// tracked by vmcnt; the caller waits for vmcnt 0 and barriers before reading
// the data.
//
// Issued from inline asm on purpose: when the compiler sees an LDS DMA in
// flight it cannot tell which LDS bytes it writes, so it makes every later
// LDS read of the wave wait for vmcnt 0 first, which turns a prefetch one tile
// ahead into a synchronous load at the next step. The compiler does not count
// these loads in its own vmcnt bookkeeping; as vector memory operations
// complete in issue order that only makes its own waits stricter.
// M0 holds the LDS address (bound as an operand, so the compiler writes it);
// an SALU write of M0 needs one wait state before an LDS DMA reads it.
__device__ __forceinline__ void load_lds16(const void* src, void* lds_wave_base) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds_wave_base);
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "{m0}"(m0)
               : "memory");
}

// Workgroup barrier that orders LDS accesses only. __syncthreads() fences
// every address space, which makes each wave wait for all of its global loads
// (vmcnt 0) first; prefetches in flight then stall every step that has a
// barrier. This one waits for the wave's LDS accesses alone, so loads issued
// earlier (global_load_lds included, which the caller waits for explicitly
// before reading what they wrote) keep flying across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ------------------------------------------------------------- forward step
// One timestep of the recurrence on a thread's 2x4 block: S0/S1 are rows 2q
// and 2q+1, columns 4L .. 4L+3; w4, a4, b4, k4, r4 hold those columns of w~,
// a, b, k, r and v the two rows of v (wkv7_common/kernel.rs:66-87):
//   sa_j = sum_i a_i S[j,i];  S[j,i] = (S[j,i] w~_i + sa_j b_i) + k_i v_j;
//   y_j = sum_i S[j,i] r_i.
// On return sa0/sa1 hold sa of both rows in every lane and y holds y of row
// 2q in lanes 0-7 and of row 2q+1 in lanes 8-15 of the DPP row.
__device__ __forceinline__ void fwd_step(float* S0, float* S1, float4 w4, float4 a4,
                                         float4 b4, float4 k4, float4 r4, float2 v, int L,
                                         float& sa0, float& sa1, float& y) {
  const float w[4] = {w4.x, w4.y, w4.z, w4.w}, a[4] = {a4.x, a4.y, a4.z, a4.w};
  const float b[4] = {b4.x, b4.y, b4.z, b4.w}, k[4] = {k4.x, k4.y, k4.z, k4.w};
  const float r[4] = {r4.x, r4.y, r4.z, r4.w};
  float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    p0 = __builtin_fmaf(a[c], S0[c], p0);
    p1 = __builtin_fmaf(a[c], S1[c], p1);
  }
  row16_sum2(p0, p1, L);
  sa0 = p0;
  sa1 = p1;
  float yy[2] = {0.0f, 0.0f};
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    S0[c] = __builtin_fmaf(k[c], v.x, __builtin_fmaf(b[c], sa0, S0[c] * w[c]));
    S1[c] = __builtin_fmaf(k[c], v.y, __builtin_fmaf(b[c], sa1, S1[c] * w[c]));
    yy[0] = __builtin_fmaf(r[c], S0[c], yy[0]);
    yy[1] = __builtin_fmaf(r[c], S1[c], yy[1]);
  }
  row16_scatter<2>(yy, L);
  y = yy[0];
}

}  // namespace wkv7
