// The language model's loss: cross entropy of the next-token logits with
// l2wrap's gradient term (examples/rwkv-lm/src/model.rs:158-169,
// kernels/l2wrap/mod.rs:38-66), one forward and one backward pass over the
// logits instead of a cast to fp32, a softmax, its backward, a cast back and
// l2wrap's max / clone / scatter.
//
// One block of 256 threads per row. Each thread walks the row in pieces of 8
// logits (one 16-byte access for bf16 when the vocabulary is a multiple of 8,
// else element by element), keeping a running maximum m, the sum
// s of exp(x - m) rescaled whenever m grows, and the first index of m. The
// 256 partial (m, s, index) triples are combined by wave shuffles and then
// across the four waves in a fixed order, so a row's result does not depend
// on scheduling. The backward recomputes exp(x - lse) from the saved
// log-sum-exp and writes each gradient once.
#include <cmath>
#include <climits>

#include "lm_loss_launch.hpp"

namespace rwkv_loss {
namespace {

struct Piece {
  float v[kPiece];
};

template <bool BF>
__device__ __forceinline__ Piece load_piece(const void* base, int64_t i) {
  Piece p;
  if constexpr (BF) {
    const uint4 raw = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + i);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      p.v[2 * k] = __builtin_bit_cast(float, w[k] << 16);
      p.v[2 * k + 1] = __builtin_bit_cast(float, w[k] & 0xffff0000u);
    }
  } else {
    const float4* f = reinterpret_cast<const float4*>(static_cast<const float*>(base) + i);
    const float4 a = f[0], b = f[1];
    p.v[0] = a.x; p.v[1] = a.y; p.v[2] = a.z; p.v[3] = a.w;
    p.v[4] = b.x; p.v[5] = b.y; p.v[6] = b.z; p.v[7] = b.w;
  }
  return p;
}

template <bool BF>
__device__ __forceinline__ void store_piece(void* base, int64_t i, const Piece& p) {
  if constexpr (BF) {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      w[k] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(p.v[2 * k]))) |
             (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(p.v[2 * k + 1])))
              << 16);
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(base) + i) = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
    float4* f = reinterpret_cast<float4*>(static_cast<float*>(base) + i);
    f[0] = make_float4(p.v[0], p.v[1], p.v[2], p.v[3]);
    f[1] = make_float4(p.v[4], p.v[5], p.v[6], p.v[7]);
  }
}

// logits j0 .. j0 + 7 of a row: one vector access when every row is a whole
// number of pieces (VEC), else element by element, -inf past the row's end
template <bool BF, bool VEC>
__device__ __forceinline__ Piece load_row(const void* base, int64_t row0, int64_t j0, int64_t V) {
  if constexpr (VEC) {
    return load_piece<BF>(base, row0 + j0);
  } else {
    Piece p;
#pragma unroll
    for (int k = 0; k < kPiece; ++k) {
      const int64_t j = j0 + k;
      p.v[k] = j >= V ? -INFINITY
               : BF   ? __builtin_bit_cast(float, static_cast<uint32_t>(
                                                    static_cast<const uint16_t*>(base)[row0 + j])
                                                    << 16)
                      : static_cast<const float*>(base)[row0 + j];
    }
    return p;
  }
}

template <bool BF, bool VEC>
__device__ __forceinline__ void store_row(void* base, int64_t row0, int64_t j0, int64_t V,
                                          const Piece& p) {
  if constexpr (VEC) {
    store_piece<BF>(base, row0 + j0, p);
  } else {
#pragma unroll
    for (int k = 0; k < kPiece; ++k) {
      const int64_t j = j0 + k;
      if (j >= V) break;
      if constexpr (BF)
        static_cast<uint16_t*>(base)[row0 + j] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(p.v[k]));
      else
        static_cast<float*>(base)[row0 + j] = p.v[k];
    }
  }
}

// running (max, sum of exp(x - max), first index of max)
struct Run {
  float m, s;
  int idx;
};

__device__ __forceinline__ float scaled(float s, float m, float to) {
  return s == 0.f ? 0.f : s * __expf(m - to);
}

// b covers indices after a's when they come from one thread; across threads
// the smaller index wins a tie
__device__ __forceinline__ Run combine(const Run& a, const Run& b) {
  Run r;
  r.m = fmaxf(a.m, b.m);
  r.s = scaled(a.s, a.m, r.m) + scaled(b.s, b.m, r.m);
  r.idx = a.m > b.m ? a.idx : b.m > a.m ? b.idx : min(a.idx, b.idx);
  return r;
}

template <bool BF, bool VEC>
__global__ __launch_bounds__(kThreads) void xent_forward_kernel(XentArgs a) {
  __shared__ Run part[kThreads / 64];
  const int64_t row = blockIdx.x;
  const int64_t V = a.vocab, base = row * V, pieces = (V + kPiece - 1) / kPiece;
  Run run{-INFINITY, 0.f, INT_MAX};
  for (int64_t q = threadIdx.x; q < pieces; q += kThreads) {
    const Piece p = load_row<BF, VEC>(a.logits, base, q * kPiece, V);
    float cm = p.v[0];
    int ci = 0;
#pragma unroll
    for (int k = 1; k < kPiece; ++k)
      if (p.v[k] > cm) {
        cm = p.v[k];
        ci = k;
      }
    const float m = fmaxf(run.m, cm);
    float s = scaled(run.s, run.m, m);
#pragma unroll
    for (int k = 0; k < kPiece; ++k) s += __expf(p.v[k] - m);
    if (cm > run.m) run.idx = static_cast<int>(q * kPiece) + ci;
    run.m = m;
    run.s = s;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    Run o;
    o.m = __shfl_xor(run.m, off);
    o.s = __shfl_xor(run.s, off);
    o.idx = __shfl_xor(run.idx, off);
    run = combine(run, o);
  }
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = run;
  __syncthreads();
  if (threadIdx.x == 0) {
    Run r = part[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) r = combine(r, part[w]);
    const float lse = r.m + logf(r.s);
    const int64_t t = a.targets[row];
    float xt = NAN;
    if (t >= 0 && t < V)
      xt = a.bf16 ? __builtin_bit_cast(float, static_cast<uint32_t>(
                                                  static_cast<const uint16_t*>(a.logits)[base + t])
                                                  << 16)
                  : static_cast<const float*>(a.logits)[base + t];
    a.row_loss[row] = lse - xt;
    a.row_lse[row] = lse;
    a.row_max[row] = r.m;
    a.row_argmax[row] = r.idx;
  }
}

template <bool BF, bool VEC>
__global__ __launch_bounds__(kThreads) void xent_backward_kernel(XentArgs a) {
  const int64_t row = blockIdx.x;
  const int64_t V = a.vocab, base = row * V, pieces = (V + kPiece - 1) / kPiece;
  const float lse = a.lse[row], g = a.row_grad[row];
  const float l2 = a.l2wrap_scale * a.max[row];
  const int64_t t = a.targets[row], am = a.argmax[row];
  for (int64_t q = threadIdx.x; q < pieces; q += kThreads) {
    Piece p = load_row<BF, VEC>(a.logits, base, q * kPiece, V);
    const int64_t j0 = q * kPiece;
#pragma unroll
    for (int k = 0; k < kPiece; ++k) {
      float d = g * __expf(p.v[k] - lse);
      if (j0 + k == t) d -= g;
      if (j0 + k == am) d += l2;
      p.v[k] = d;
    }
    store_row<BF, VEC>(a.logits_grad, base, q * kPiece, V, p);
  }
}

template <typename K>
hipError_t launch(K kernel, const XentArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(a.rows)), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_xent_forward(const XentArgs& a, hipStream_t s) {
  if (a.rows == 0) return hipSuccess;
  if (a.vocab % kPiece == 0)
    return a.bf16 ? launch(xent_forward_kernel<true, true>, a, s)
                  : launch(xent_forward_kernel<false, true>, a, s);
  return a.bf16 ? launch(xent_forward_kernel<true, false>, a, s)
                : launch(xent_forward_kernel<false, false>, a, s);
}

hipError_t launch_xent_backward(const XentArgs& a, hipStream_t s) {
  if (a.rows == 0) return hipSuccess;
  if (a.vocab % kPiece == 0)
    return a.bf16 ? launch(xent_backward_kernel<true, true>, a, s)
                  : launch(xent_backward_kernel<false, true>, a, s);
  return a.bf16 ? launch(xent_backward_kernel<true, false>, a, s)
                : launch(xent_backward_kernel<false, false>, a, s);
}

}  // namespace rwkv_loss
