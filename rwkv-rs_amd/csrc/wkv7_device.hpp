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
//
// Lane-relative row order. Lanes 8-15 of each DPP row (up = 1) keep their row
// pair swapped: a thread's "own" row is 2q + up, its "other" row 2q + 1 - up,
// and every per-row quantity it holds (state rows, row operands, partial
// sums) is ordered (own, other). The first level of a sum over the DPP row
// pairs lane L with L ^ 8, whose own row is this lane's other row, so it adds
// the partner's "other" value to the own value with no select; the remaining
// levels run inside an 8-lane half, where every lane has the same own row.
// With the plain order, every reduce-scatter level needs two v_cndmask per
// value pair to choose what to keep and what to send.
//
// Sums that are outputs only (y in the forward, the six gradients in the
// backward) are not on the recurrence's dependency chain: their partials stay
// in registers for a whole LDS tile of timesteps and are reduced in one batch
// at the tile end, where the independent DPP chains overlap each other.
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
  // one value into a staging buffer of this type; 4 staged values to memory
  static __device__ __forceinline__ void put1(float* p, float x) { *p = x; }
  static __device__ __forceinline__ void copy4(float* dst, const float* src) {
    *reinterpret_cast<float4*>(dst) = *reinterpret_cast<const float4*>(src);
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
  static __device__ __forceinline__ void put1(bf16_t* p, float x) { *p = (bf16_t)f32_to_bf16(x); }
  static __device__ __forceinline__ void copy4(bf16_t* dst, const bf16_t* src) {
    *reinterpret_cast<uint2*>(dst) = *reinterpret_cast<const uint2*>(src);
  }
};

// decay w~ = exp(W_SCALE * sigmoid(x)), kernel.rs:63-65; also sigmoid(x)
__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float decay_f(float sig) { return expf(kWScale * sig); }

// ------------------------------------------------------- cross-lane reduction
// DPP move feeding an add (the compiler fuses the pair into v_add_f32_dpp)
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
// DPP move whose result is used on its own. Every pattern used here reads a
// lane of the same row for every lane, so no lane keeps an "old" value and
// none needs to be materialised.
template <int CTRL>
__device__ __forceinline__ float dpp_get(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(
      __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, true));
}

// DPP controls used below. row_ror:8 pairs lane L with L ^ 8 (the other half
// of the 16-lane DPP row), row_half_mirror pairs L with 7 - L inside an 8-lane
// half, the quad permutations pair L with L ^ 2 and L ^ 1.
constexpr int kDppRor8 = 0x128;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppQuadSwap2 = 0x4E;   // quad_perm:[2,3,0,1]
constexpr int kDppQuadSwap1 = 0xB1;   // quad_perm:[1,0,3,2]

// One recursive-halving step of a reduce-scatter: the lane keeps half of its
// N values (the upper half when `upper`) and adds the partner's copy of that
// half; the partner lane (the DPP source) has the opposite `upper`.
template <int CTRL, int N>
__device__ __forceinline__ void rs_step(float* x, bool upper) {
#pragma unroll
  for (int j = 0; j < N / 2; ++j) {
    const float keep = upper ? x[N / 2 + j] : x[j];
    const float send = upper ? x[j] : x[N / 2 + j];
    x[j] = keep + dpp_mov<CTRL>(send);
  }
}

// Full sums over the DPP row of a pair of per-row partial sums (own, other):
// on return `own` and `other` hold the sums of the thread's own and other
// row, in every lane. Select-free: lane L ^ 8's other row is this lane's own
// row, and after the first level all lanes of a half hold the same row.
__device__ __forceinline__ void row_pair_sum(float& own, float& other) {
  float s = own + dpp_mov<kDppRor8>(other);
  s += dpp_mov<kDppHalfMirror>(s);
  s += dpp_mov<kDppQuadSwap2>(s);
  s += dpp_mov<kDppQuadSwap1>(s);
  own = s;
  other = dpp_get<kDppRor8>(s);
}

// Reduce-scatter over the DPP row of N per-row partial sums (N a multiple of
// 16) laid out as [own block | other block], value m of the other block
// belonging to the other row as value m of the own block does to the own row.
// Afterwards x[0 .. N/16 - 1] of lane L hold the full sums of the own-block
// values (L & 7) * N/16 .. (L & 7) * N/16 + N/16 - 1 (of the lane's own row).
// The first level is select-free (see row_pair_sum); the three levels inside
// an 8-lane half use rs_step.
// Level `lv` (0..3) of row16_reduce_scatter alone, so that the levels of one
// batch can be spread over independent work.
template <int N, int lv>
__device__ __forceinline__ void row16_rs_level(float* x, int L) {
  static_assert(N % 16 == 0, "N must be a multiple of 16");
  if constexpr (lv == 0) {
#pragma unroll
    for (int j = 0; j < N / 2; ++j) x[j] += dpp_mov<kDppRor8>(x[N / 2 + j]);
  } else if constexpr (lv == 1) {
    rs_step<kDppHalfMirror, N / 2>(x, (L & 4) != 0);
  } else if constexpr (lv == 2) {
    rs_step<kDppQuadSwap2, N / 4>(x, (L & 2) != 0);
  } else {
    rs_step<kDppQuadSwap1, N / 8>(x, (L & 1) != 0);
  }
}

template <int N>
__device__ __forceinline__ void row16_reduce_scatter(float* x, int L) {
  row16_rs_level<N, 0>(x, L);
  row16_rs_level<N, 1>(x, L);
  row16_rs_level<N, 2>(x, L);
  row16_rs_level<N, 3>(x, L);
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
// One timestep of the recurrence on a thread's 2x4 block (wkv7_common/
// kernel.rs:66-87): So/St are the own and other row, columns 4L .. 4L+3;
// w4, a4, b4, k4, r4 hold those columns of w~, a, b, k, r and v = (v_own,
// v_other):
//   sa_j = sum_i a_i S[j,i];  S[j,i] = (S[j,i] w~_i + sa_j b_i) + k_i v_j;
//   y_j = sum_i S[j,i] r_i.
// On return sa_o/sa_t hold sa of the own and other row (every lane) and
// yp_o/yp_t the thread's partial y sums over its four columns; the caller
// reduces those over the DPP row (they are not needed by the next step).
__device__ __forceinline__ void fwd_step(float* So, float* St, float4 w4, float4 a4, float4 b4,
                                         float4 k4, float4 r4, float2 v, float& sa_o,
                                         float& sa_t, float& yp_o, float& yp_t) {
  const float w[4] = {w4.x, w4.y, w4.z, w4.w}, a[4] = {a4.x, a4.y, a4.z, a4.w};
  const float b[4] = {b4.x, b4.y, b4.z, b4.w}, k[4] = {k4.x, k4.y, k4.z, k4.w};
  const float r[4] = {r4.x, r4.y, r4.z, r4.w};
  // partial sums start from their first product (a product, not an FMA with
  // +0, which the compiler must keep as a three-operand VOP3 FMA)
  float po = a[0] * So[0], pt = a[0] * St[0];
#pragma unroll
  for (int c = 1; c < 4; ++c) {
    po = __builtin_fmaf(a[c], So[c], po);
    pt = __builtin_fmaf(a[c], St[c], pt);
  }
  row_pair_sum(po, pt);
  sa_o = po;
  sa_t = pt;
  float yo, yt;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    So[c] = __builtin_fmaf(k[c], v.x, __builtin_fmaf(b[c], sa_o, So[c] * w[c]));
    St[c] = __builtin_fmaf(k[c], v.y, __builtin_fmaf(b[c], sa_t, St[c] * w[c]));
    yo = c == 0 ? r[c] * So[c] : __builtin_fmaf(r[c], So[c], yo);
    yt = c == 0 ? r[c] * St[c] : __builtin_fmaf(r[c], St[c], yt);
  }
  yp_o = yo;
  yp_t = yt;
}

// ------------------------------------------------------ bf16 arithmetic
// one bf16 operation: an fp32 result of bf16 operands rounded to bf16 (ties
// to even). Products of two bf16 values are exact in fp32, and a sum rounded
// to fp32 and then to bf16 equals the sum rounded once (fp32 carries more
// than twice bf16's significand bits plus two).
__device__ __forceinline__ float rb(float x) { return (float)(__bf16)x; }

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
// rb(x) + rb(p) as an fp32 sum: both roundings in one packed conversion, the
// sum of the two bf16 halves by a bf16 dot product with (1, 1). Three
// instructions where rounding both operands and adding takes five (the
// conversion, the zeroed accumulator and the dot product against two
// conversions, two widenings and the addition). Every caller rounds the
// result to bf16 (rb, or the next add_rb), and that rounding equals the
// rounding of the IEEE fp32 addition of the two halves. The fp32 sum itself
// is not always IEEE's: measured, when one addend is below 2^-16 of the
// other it can be one fp32 ulp off. That cannot move the bf16 rounding:
// with e the sum's exponent, a bf16 midpoint is then at least
// 2^(e-8) - 2^(e-15) from the exact sum, and for every other pair the sum
// and the midpoints lie on the 2^(e-23) grid. Subnormal results are kept;
// (-0) + (-0) gives +0 (the +0 accumulator). tests/test_gpu_selftest.py
// holds these facts on the device.
__device__ __forceinline__ float add_rb(float x, float p) {
  const bf16x2_t h = __builtin_convertvector(f32x2_t{x, p}, bf16x2_t);
  return __builtin_amdgcn_fdot2_f32_bf16(h, bf16x2_t{(__bf16)1.0f, (__bf16)1.0f}, 0.0f, false);
}


}  // namespace wkv7
