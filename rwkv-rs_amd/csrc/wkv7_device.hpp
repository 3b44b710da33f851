// Device-side building blocks shared by the WKV7 kernels (gfx950 / CDNA4).
//
// Work layout (all three kernels). One workgroup of 256 threads (4 wave64)
// owns one (batch, head) pair and its 64x64 fp32 state. Inside a wave the
// lanes form four 16-lane DPP rows. A DPP row is four quads. With
//   wave = tid / 64, g = (tid % 64) / 16, L = tid % 16, lo = L % 4, hi = L / 4
// a thread's "own index" is e = 16*wave + 4*g + lo (0..63) and its "segment"
// is hi (0..3, covering indices 16*hi .. 16*hi+15). The forward kernel keeps
// state row e, columns 16*hi+m (m = 0..15) in 16 VGPRs.
//
// Per-timestep vectors (one value per index 0..63) are stored in LDS as fp32
// and read with one ds_read_b128 per lane: lane L of every DPP row reads
// elements 4L..4L+3. Element 16*hi+m of a vector then sits in quad hi, quad
// lane m/4, component m%4, so a quad_perm:[s,s,s,s] DPP source operand hands
// element 16*hi+4s+c to all four lanes of the quad in the same instruction
// that consumes it. That turns the "broadcast a column value to every row"
// of the recurrence into a free operand modifier instead of an LDS read per
// element. The compiler does not fold DPP moves into v_fmac_f32, so the
// element loops are short inline-asm blocks of v_fmac_f32_dpp/v_mul_f32_dpp.
//
// DPP hazard: on gfx9 a DPP instruction that reads a VGPR written by a VALU
// instruction less than two instructions earlier reads a stale value. Every
// asm block starts with `s_nop 1`, and inside a block no DPP source operand is
// ever written, so the blocks are safe whatever the compiler schedules before
// them. The cross-lane reductions use the __builtin_amdgcn_update_dpp path,
// for which the compiler inserts the wait states itself.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wkv7 {

constexpr int kHead = 64;        // head size N (the kernels are specialised)
constexpr int kThreads = 256;    // 4 waves per (batch, head)
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
// Sum over the four lanes L, L+4, L+8, L+12 of a DPP row (the four segments
// of one index). The result is bit-identical in all four lanes: the first
// step pairs segments {0,2} and {1,3}, the second adds the two pair sums, and
// IEEE addition is commutative.
__device__ __forceinline__ float seg_sum(float x) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
           0, __builtin_bit_cast(int, x), 0x128 /* row_ror:8 */, 0xf, 0xf, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
           0, __builtin_bit_cast(int, x), 0x124 /* row_ror:4 */, 0xf, 0xf, false));
  return x;
}

// ------------------------------------------------------------ asm helpers
#define WKV7_QP(s) " quad_perm:[" #s "," #s "," #s "," #s "] row_mask:0xf bank_mask:0xf\n\t"

// ------------------------------------------- forward step (rows independent)
// sa0/sa1 += a[m] * S[m] over the 16 columns m of this thread's segment
// (a quad-broadcast: column 16*hi+4s+c is component c of quad lane s)
__device__ __forceinline__ void fwd_sa16(float& sa0, float& sa1, float4 a, const float* S) {
  asm("s_nop 1\n\t"
      "v_fmac_f32_dpp %0, %2, %6" WKV7_QP(0)
      "v_fmac_f32_dpp %1, %3, %7" WKV7_QP(0)
      "v_fmac_f32_dpp %0, %4, %8" WKV7_QP(0)
      "v_fmac_f32_dpp %1, %5, %9" WKV7_QP(0)
      "v_fmac_f32_dpp %0, %2, %10" WKV7_QP(1)
      "v_fmac_f32_dpp %1, %3, %11" WKV7_QP(1)
      "v_fmac_f32_dpp %0, %4, %12" WKV7_QP(1)
      "v_fmac_f32_dpp %1, %5, %13" WKV7_QP(1)
      "v_fmac_f32_dpp %0, %2, %14" WKV7_QP(2)
      "v_fmac_f32_dpp %1, %3, %15" WKV7_QP(2)
      "v_fmac_f32_dpp %0, %4, %16" WKV7_QP(2)
      "v_fmac_f32_dpp %1, %5, %17" WKV7_QP(2)
      "v_fmac_f32_dpp %0, %2, %18" WKV7_QP(3)
      "v_fmac_f32_dpp %1, %3, %19" WKV7_QP(3)
      "v_fmac_f32_dpp %0, %4, %20" WKV7_QP(3)
      "v_fmac_f32_dpp %1, %5, %21" WKV7_QP(3)
      : "+v"(sa0), "+v"(sa1)
      : "v"(a.x), "v"(a.y), "v"(a.z), "v"(a.w), "v"(S[0]), "v"(S[1]), "v"(S[2]),
        "v"(S[3]), "v"(S[4]), "v"(S[5]), "v"(S[6]), "v"(S[7]), "v"(S[8]), "v"(S[9]),
        "v"(S[10]), "v"(S[11]), "v"(S[12]), "v"(S[13]), "v"(S[14]), "v"(S[15]));
}

// For the 8 columns m = 4*S0 .. 4*S0+7 (quad lanes S0 and S0+1):
//   S[m] = S[m] * w~ + sa * b + k * v_e ;  y0/y1 += r * S[m]
// in the reference's operation order ((S*w + sa*b) + k*v, kernel.rs:79-83).
#define WKV7_DEF_FWD_UPD8(S0, S1)                                                   \
  __device__ __forceinline__ void fwd_upd8_q##S0(float* s, float& y0, float& y1,     \
                                                 float4 w, float4 b, float4 k,       \
                                                 float4 r, float sa, float ve) {     \
    asm("s_nop 1\n\t"                                                                \
        "v_mul_f32_dpp %0, %10, %0" WKV7_QP(S0)                                      \
        "v_mul_f32_dpp %1, %11, %1" WKV7_QP(S0)                                      \
        "v_mul_f32_dpp %2, %12, %2" WKV7_QP(S0)                                      \
        "v_mul_f32_dpp %3, %13, %3" WKV7_QP(S0)                                      \
        "v_mul_f32_dpp %4, %10, %4" WKV7_QP(S1)                                      \
        "v_mul_f32_dpp %5, %11, %5" WKV7_QP(S1)                                      \
        "v_mul_f32_dpp %6, %12, %6" WKV7_QP(S1)                                      \
        "v_mul_f32_dpp %7, %13, %7" WKV7_QP(S1)                                      \
        "v_fmac_f32_dpp %0, %14, %26" WKV7_QP(S0)                                    \
        "v_fmac_f32_dpp %1, %15, %26" WKV7_QP(S0)                                    \
        "v_fmac_f32_dpp %2, %16, %26" WKV7_QP(S0)                                    \
        "v_fmac_f32_dpp %3, %17, %26" WKV7_QP(S0)                                    \
        "v_fmac_f32_dpp %4, %14, %26" WKV7_QP(S1)                                    \
        "v_fmac_f32_dpp %5, %15, %26" WKV7_QP(S1)                                    \
        "v_fmac_f32_dpp %6, %16, %26" WKV7_QP(S1)                                    \
        "v_fmac_f32_dpp %7, %17, %26" WKV7_QP(S1)                                    \
        "v_fmac_f32_dpp %0, %18, %27" WKV7_QP(S0)                                    \
        "v_fmac_f32_dpp %1, %19, %27" WKV7_QP(S0)                                    \
        "v_fmac_f32_dpp %2, %20, %27" WKV7_QP(S0)                                    \
        "v_fmac_f32_dpp %3, %21, %27" WKV7_QP(S0)                                    \
        "v_fmac_f32_dpp %4, %18, %27" WKV7_QP(S1)                                    \
        "v_fmac_f32_dpp %5, %19, %27" WKV7_QP(S1)                                    \
        "v_fmac_f32_dpp %6, %20, %27" WKV7_QP(S1)                                    \
        "v_fmac_f32_dpp %7, %21, %27" WKV7_QP(S1)                                    \
        "v_fmac_f32_dpp %8, %22, %0" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %9, %23, %1" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %8, %24, %2" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %9, %25, %3" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %8, %22, %4" WKV7_QP(S1)                                     \
        "v_fmac_f32_dpp %9, %23, %5" WKV7_QP(S1)                                     \
        "v_fmac_f32_dpp %8, %24, %6" WKV7_QP(S1)                                     \
        "v_fmac_f32_dpp %9, %25, %7" WKV7_QP(S1)                                     \
        : "+v"(s[0]), "+v"(s[1]), "+v"(s[2]), "+v"(s[3]), "+v"(s[4]), "+v"(s[5]),   \
          "+v"(s[6]), "+v"(s[7]), "+v"(y0), "+v"(y1)                                 \
        : "v"(w.x), "v"(w.y), "v"(w.z), "v"(w.w), "v"(b.x), "v"(b.y), "v"(b.z),      \
          "v"(b.w), "v"(k.x), "v"(k.y), "v"(k.z), "v"(k.w), "v"(r.x), "v"(r.y),      \
          "v"(r.z), "v"(r.w), "v"(sa), "v"(ve));                                     \
  }
WKV7_DEF_FWD_UPD8(0, 1)
WKV7_DEF_FWD_UPD8(2, 3)

}  // namespace wkv7
