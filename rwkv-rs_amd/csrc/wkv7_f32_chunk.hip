// Chunked WKV7 on the fp32 matrix cores (fp32 operands, fp32 products).
//
// Computes what wkv7_forward_kernel and wkv7_backward_kernel do
// (crates/rwkv-nn/src/kernels/wkv7_common/kernel.rs:6-114 and 116-308,
// launched by wkv7_common/host.rs:29-183 and 185-369) for fp32 operands at
// chunk lengths that are multiples of 16 (and the forward of bf16 operands,
// widened to fp32 as the reference casts them; the launchers' comments say
// where each kernel is picked), with every product an fp32
// product: the chunked matrix form of wkv7_chunk.hpp (the same identities as
// the bf16 kernels) on v_mfma_f32_16x16x4_f32, which multiplies fp32 values
// in fp32 and sums in fp32. The decays are formed as the reference forms them,
// w~ = exp(W_SCALE * sigmoid(x)) with sigmoid(x) = 1 / (1 + exp(-x)), and
// multiplied up within a chunk by a scan across the 16 lanes of a row
// (gamma_t = w~_0 ... w~_t, four fp32 multiplications deep). The reference's
// step-by-step recurrence never forms these products; it multiplies the state
// by one w~ per step. The two orders round differently, inside the fp32 bar
// (tests/test_gpu_parity.py).
//
// Matrix-core layout (v_mfma_f32_16x16x4_f32, lane l, quad qd = l / 16,
// t = l % 16): MFMA number r (r < 4) of a 16x16x16 product reads
//   A operand  lane l: A[m = t][k = 4 qd + r]
//   B operand  lane l: B[k = 4 qd + r][n = t]
// and the result is D[m = 4 qd + r][n = t] in register r. A result tile is
// therefore directly the B operand of a product that contracts over its rows,
// and, read as an A operand, it is its own transpose. The state is held in
// that layout, as 4 tiles of rows = key i (16 ib + 4 qd + r), columns =
// value j (16 jb + t), so it is the B operand of every contraction over
// keys without a transpose.
#include <type_traits>

#include "wkv7_chunk.hpp"
#include "wkv7_launch.hpp"

namespace wkv7 {
namespace {

using namespace chunk;

constexpr int kBlock = 512;      // 8 waves per (batch, head)
constexpr int kLd = 68;          // padded fp32 row: rows 4 banks apart
constexpr int kLg = 20;          // padded 16-wide rows of the 16x16 products
enum { R_X, R_R, R_K, R_V, R_A, R_B, R_COUNT };          // raw chunk rows
enum { D_AH, D_RH, D_KT, D_BT, D_KE, D_BE, D_COUNT };    // decayed rows
enum { G_AB, G_AK, G_RB, G_RK, G_COUNT };                // 16x16 step products

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
// D += A B for one 16x16x16 block: a[r] = A[t][4 qd + r], b[r] = B[4 qd + r][t]
__device__ __forceinline__ f32x4 mm16(f32x4 a, f32x4 b, f32x4 c) {
#pragma unroll
  for (int r = 0; r < 4; ++r) c = mfma4(a[r], b[r], c);
  return c;
}
// A-operand fragment of rows [16][kLd] (row t, keys k0 + 4 qd ..): one
// 16-byte read; rows 4 banks apart, so the 16 rows hit distinct banks
__device__ __forceinline__ f32x4 row4(const float* tile, int ld, int t, int k0, int qd) {
  return *reinterpret_cast<const f32x4*>(tile + t * ld + k0 + 4 * qd);
}
// B-operand fragment read down a column: tile[4 qd + r][c]
__device__ __forceinline__ f32x4 col4(const float* tile, int ld, int c, int qd) {
  return f32x4{tile[(4 * qd) * ld + c], tile[(4 * qd + 1) * ld + c], tile[(4 * qd + 2) * ld + c],
               tile[(4 * qd + 3) * ld + c]};
}
// X (rows t, 64 columns) times Z^T (rows n, 64 columns): 16 x 16 over 64
__device__ __forceinline__ f32x4 gram64(const float* X, const float* Z, int t, int qd) {
  f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) c = mm16(row4(X, kLd, t, 16 * kk, qd), row4(Z, kLd, t, 16 * kk, qd), c);
  return c;
}
// inclusive product over the 16 lanes of a DPP row (lane t: x_0 ... x_t)
__device__ __forceinline__ float row_prod16(float x) {
  auto sh = [](float v, auto ctrl) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
        __builtin_bit_cast(int, 1.0f), __builtin_bit_cast(int, v), decltype(ctrl)::value, 0xf, 0xf, false));
  };
  x *= sh(x, std::integral_constant<int, 0x111>{});   // row_shr:1
  x *= sh(x, std::integral_constant<int, 0x112>{});   // row_shr:2
  x *= sh(x, std::integral_constant<int, 0x114>{});   // row_shr:4
  x *= sh(x, std::integral_constant<int, 0x118>{});   // row_shr:8
  return x;
}
// the previous lane's value in the DPP row, 1 in lane 0
__device__ __forceinline__ float row_prev16(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      __builtin_bit_cast(int, 1.0f), __builtin_bit_cast(int, x), 0x111, 0xf, 0xf, false));
}

// P = (I - A)^-1 for A strictly lower triangular (A^16 = 0), as
// (I + A)(I + A^2)(I + A^4)(I + A^8). Every factor is kept with its
// transpose, both in the result layout, because a product X Y takes X^T's
// result registers as its A operand: MM(U, V) = U^T V for result tiles U, V.
// Returns P and its transpose.
__device__ __forceinline__ f32x4 MM(f32x4 u, f32x4 v) { return mm16(u, v, f32x4{0.f, 0.f, 0.f, 0.f}); }
__device__ __forceinline__ void unit_lower_inverse_f32(f32x4 a, f32x4 at, int t, int qd, f32x4& p,
                                                       f32x4& pt) {
  f32x4 id;
#pragma unroll
  for (int r = 0; r < 4; ++r) id[r] = (4 * qd + r == t) ? 1.0f : 0.0f;
  const f32x4 a2 = MM(at, a), a2t = MM(a, at);
  const f32x4 a4 = MM(a2t, a2), a4t = MM(a2, a2t);
  const f32x4 a8 = MM(a4t, a4);
  const f32x4 q1 = id + a, q1t = id + at;
  const f32x4 q2 = q1 + MM(q1t, a2), q2t = q1t + MM(a2, q1t);
  const f32x4 q3 = q2 + MM(q2t, a4), q3t = q2t + MM(a4, q2t);
  p = q3 + MM(q3t, a8);
  pt = q3t + MM(a8, q3t);
}

// ------------------------------------------------------------------ forward
//
// One workgroup of eight waves per (batch, head), two per SIMD, in two groups
// that run concurrently and hand chunks over through LDS, as the bf16 chunked
// forward does:
//   prep waves 4-7  wave 4 + s prepares chunks c = s, s + 4, ... on its own,
//                   from registers: the chunk's rows arrive as the fragments
//                   the matrix cores read (step t, keys 16 kk + 4 qd ..; V
//                   down its columns), loaded during the previous chunk it
//                   prepared. It forms the decayed rows, the four step
//                   products, P, W = P A^ and U = (P A_ak) V, and writes every
//                   operand the chain needs to slot s; it leaves the x rows of
//                   its next chunk c + 4 beside them; then it marks the slot
//                   ready;
//   chain waves 0-3 take the chunks in order; wave w owns value columns
//                   16 w .. 16 w + 15 of the state, loads chunk c's operands
//                   from slot c % 4 (one 16-byte load per fragment), computes
//                   SA, Y and the next state, turns the x rows of chunk c + 4
//                   of keys 16 w .. 16 w + 15 into gamma_t in place (their
//                   matrix-core work leaves the vector units idle), and marks
//                   the slot taken.
// A prep wave overwrites its slot only after all four chain waves have taken
// the chunk in it. Every wait is bounded; a wave that gives up raises the
// workgroup's fault flag, and after a final barrier the workgroup overwrites
// its (batch, head)'s outputs with NaN and counts the event in the chunked
// forwards' device counter (wkv7_take_faults).
constexpr int kChainWaves = 4;   // value tile = wave
constexpr int kSlots = 4;        // operand slots = prep waves
constexpr int kLs = 20;          // padded 16-step rows of the key-major tiles

// Operands of one chunk, in the order the chain waves load them ([lane]
// last), or as key-major tiles ([key][step]) that a chain lane reads 16 bytes
// at a time
struct F32ChunkOps {
  f32x4 w[4][64];          // W = P A^ per key tile: W[t][16 ib + 4 qd + r]
  f32x4 rh[4][64];         // R^ per key tile: R^[t][16 ib + 4 qd + r]
  f32x4 ark[64];           // A_rk[t][4 qd + r]
  f32x4 arb[64];           // A_rb[t][4 qd + r]
  f32x4 v[4][64];          // V per value tile: V[4 qd + r][16 vb + t]
  f32x4 u[4][64];          // U per value tile, result layout
  float ke[64 * kLs];      // K- = K~ gamma_L, [key][step]
  float be[64 * kLs];      // B- = B~ gamma_L, [key][step]
  float gl[64];            // gamma_L
};
// the x rows of a slot's next chunk, then (in place) its gamma_t: [step t][64
// keys], 16-byte groups g = key / 4 stored at group g ^ t so that a lane
// group's row reads and writes spread over the banks
__device__ __forceinline__ int dx_at(int t, int g) { return t * 64 + 4 * (g ^ t); }
// gamma_t of one key at step t = lane t of a DPP row: the product of the
// chunk's w~ up to t (a lane scan), w~ = exp(W_SCALE sigmoid(x))
__device__ __forceinline__ float gamma_of(float x) {
  return row_prod16(expf(kWScale * (1.0f / (1.0f + expf(-x)))));
}

// a prep wave's own LDS: the transposes of A^, A_ab and A_ak
struct F32PrepLds {
  float ah[64 * kLs];      // A^, [key][step]
  float aab[kL * kLg];     // A_ab, [t][s]
  float aak[kL * kLg];     // A_ak, [t][s]
};
// hand-over flags: ready[s] = the chunk whose operands are in slot s,
// taken[s][w] = the last chunk chain wave w loaded from slot s
struct F32Flags {
  int ready[kSlots];
  int taken[kSlots][kChainWaves];
  int fault;               // a wave gave up a wait
};

// Tin: the operand and output type, float or bf16 (bf16 rows are widened to
// fp32 exactly as they load, as the reference casts them before its kernel,
// host.rs:45-64; y is rounded to bf16 as it is stored)
template <typename Tin>
struct F32FwdParams {
  const Tin* in[R_COUNT];     // [B,T,H,64] each, in R_* order
  const float* s0;            // [B,H,64(value),64(key)] or null
  float* ckpt;                // [B,H,T/C,64(key),64(value)]
  float* sa;                  // [B,T,H,64]
  Tin* y;                     // [B,T,H,64]
  float* sT;                  // [B,H,64,64] or null
  unsigned int* faults;       // the chunked forwards' hand-over fault counter
  int T, H, C;
  uint32_t spin_limit;        // polls per hand-over wait (> 0)
};

// step t of chunk c, keys (or values) 16 kk + 4 qd .. + 3 of a row tensor:
// the A or B operand fragment of a contraction over keys. The rows are read
// once per launch, with the non-temporal hint.
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
template <typename Tin>
__device__ __forceinline__ f32x4 row_frag4(const Tin* base, int64_t tstride, int c, int t, int kk,
                                           int qd) {
  const Tin* const q = base + (int64_t)(kL * c + t) * tstride + 16 * kk + 4 * qd;
  if constexpr (std::is_same<Tin, float>::value) {
    return __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(q));
  } else {
    const u32x2 x = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(q));
    return f32x4{__uint_as_float(x[0] << 16), __uint_as_float(x[0] & 0xffff0000u),
                 __uint_as_float(x[1] << 16), __uint_as_float(x[1] & 0xffff0000u)};
  }
}
// steps 4 qd + r of chunk c, value 16 vb + t: the B operand fragment of a
// contraction over steps
template <typename Tin>
__device__ __forceinline__ f32x4 col_frag4(const Tin* base, int64_t tstride, int c, int t, int vb,
                                           int qd) {
  f32x4 x;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const Tin* const q = base + (int64_t)(kL * c + 4 * qd + r) * tstride + 16 * vb + t;
    if constexpr (std::is_same<Tin, float>::value)
      x[r] = __builtin_nontemporal_load(q);
    else
      x[r] = __uint_as_float((uint32_t)__builtin_nontemporal_load(q) << 16);
  }
  return x;
}

template <typename Tin, bool kHasS0>
__global__ __launch_bounds__(kBlock, 1) void wkv7_fwd_f32_chunk_kernel(const F32FwdParams<Tin> p) {
  __shared__ F32ChunkOps ops[kSlots];
  __shared__ F32PrepLds prep[kSlots];
  __shared__ __attribute__((aligned(16))) float dx[kSlots][kL * 64];
  __shared__ F32Flags flags;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: roles branch on it
  const int t = lane & 15, qd = lane >> 4;
  const int h = blockIdx.x, b = blockIdx.y, H = p.H, T = p.T;
  const int64_t bh = (int64_t)b * H + h;
  const int64_t tstride = (int64_t)H * kHead;
  const int64_t tok0 = ((int64_t)b * T * H + h) * kHead;
  const int nchunks = T / kL;
  const int per_ckpt = p.C / kL;
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};

  if (tid < kSlots) flags.ready[tid] = -1;
  if (tid == 0) flags.fault = 0;
  if (tid < kSlots * kChainWaves) flags.taken[tid / kChainWaves][tid % kChainWaves] = tid / kChainWaves - kSlots;
  __syncthreads();

  if (wave >= kChainWaves) {
    // ================================================= prep wave for slot s
    const int s = wave - kChainWaves;
    F32PrepLds& my = prep[s];
    if (s < nchunks) {
      const Tin* const bx = p.in[R_X] + tok0;
      const Tin* const brr = p.in[R_R] + tok0;
      const Tin* const bk = p.in[R_K] + tok0;
      const Tin* const bv = p.in[R_V] + tok0;
      const Tin* const ba = p.in[R_A] + tok0;
      const Tin* const bb = p.in[R_B] + tok0;
      // the chunk's rows: x, r, k, a, b at step t, keys 16 kk + 4 qd + r;
      // V at steps 4 qd + r, values 16 vb + t. Each register set is reloaded
      // with the wave's next chunk as soon as this chunk has consumed it.
      f32x4 X[4], R[4], K[4], A[4], Bz[4], V[4];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        X[kk] = row_frag4(bx, tstride, s, t, kk, qd);
        R[kk] = row_frag4(brr, tstride, s, t, kk, qd);
        K[kk] = row_frag4(bk, tstride, s, t, kk, qd);
        A[kk] = row_frag4(ba, tstride, s, t, kk, qd);
        Bz[kk] = row_frag4(bb, tstride, s, t, kk, qd);
        V[kk] = col_frag4(bv, tstride, s, t, kk, qd);
      }
      for (int c = s; c < nchunks; c += kSlots) {
        // the last chunk reloads itself (harmless), so the loads need no branch
        const int cn = c + kSlots < nchunks ? c + kSlots : c;
        // the slot is free once every chain wave has taken chunk c - kSlots
        bool ok = true;
        for (int w = 0; w < kChainWaves; ++w) ok &= wait_flag(&flags.taken[s][w], c - kSlots, p.spin_limit);
        if (!ok && lane == 0) lds_store_flag(&flags.fault, 1);
        lds_acquire();
        F32ChunkOps& o = ops[s];

        // decays of step t: gamma_t (formed by the chain waves, from the x rows
        // this wave left with its previous chunk; from its own registers for
        // its first chunk), gamma_{t-1}, 1 / gamma_t, gamma_L
        f32x4 gm[4];
        if (c == s) {
#pragma unroll
          for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int r = 0; r < 4; ++r) gm[kk][r] = gamma_of(X[kk][r]);
        } else {
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) gm[kk] = *reinterpret_cast<const f32x4*>(&dx[s][dx_at(t, 4 * kk + qd)]);
        }
        f32x4 gL[4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float gam = gm[kk][r];
            const float gpv = row_prev16(gam);
            const float gin = 1.0f / gam;
            gL[kk][r] = row_last16(gam);
            A[kk][r] *= gpv;     // A^
            R[kk][r] *= gam;     // R^
            K[kk][r] *= gin;     // K~
            Bz[kk][r] *= gin;    // B~
          }
        if (cn != c) {
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) X[kk] = row_frag4(bx, tstride, cn, t, kk, qd);
        }

        // the step products as row fragments: lane (qd, t) holds
        // A_xy[t][s = 4 qd + r] = x_t . y_s
        f32x4 aab = zero, aak = zero, ark = zero, arb = zero;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          aab = mm16(Bz[kk], A[kk], aab);
          aak = mm16(K[kk], A[kk], aak);
          ark = mm16(K[kk], R[kk], ark);
          arb = mm16(Bz[kk], R[kk], arb);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int sx = 4 * qd + r;
          if (!(sx < t)) { aab[r] = 0.f; aak[r] = 0.f; }
          if (!(sx <= t)) { ark[r] = 0.f; arb[r] = 0.f; }
        }
        // what the chain reads of R^, A_rk, A_rb, V, K-, B-, gamma_L
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          o.rh[kk][lane] = R[kk];
          o.v[kk][lane] = V[kk];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            o.ke[(16 * kk + 4 * qd + r) * kLs + t] = K[kk][r] * gL[kk][r];
            o.be[(16 * kk + 4 * qd + r) * kLs + t] = Bz[kk][r] * gL[kk][r];
          }
          if (t == 0) *reinterpret_cast<f32x4*>(&o.gl[16 * kk + 4 * qd]) = gL[kk];
        }
        o.ark[lane] = ark;
        o.arb[lane] = arb;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          R[kk] = row_frag4(brr, tstride, cn, t, kk, qd);
          K[kk] = row_frag4(bk, tstride, cn, t, kk, qd);
          Bz[kk] = row_frag4(bb, tstride, cn, t, kk, qd);
        }

        // A^, A_ab and A_ak transposed through the wave's own LDS
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
          for (int r = 0; r < 4; ++r) my.ah[(16 * kk + 4 * qd + r) * kLs + t] = A[kk][r];
        *reinterpret_cast<f32x4*>(&my.aab[t * kLg + 4 * qd]) = aab;
        *reinterpret_cast<f32x4*>(&my.aak[t * kLg + 4 * qd]) = aak;
        wave_lds_sync();
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) A[kk] = row_frag4(ba, tstride, cn, t, kk, qd);
        // P = (I - A_ab)^-1; its row fragments Pt[r] = P[t][4 qd + r]
        f32x4 P, Pt;
        unit_lower_inverse_f32(col4(my.aab, kLg, t, qd), aab, t, qd, P, Pt);
        // W^T tile ib = A^T P^T: result rows = keys 16 ib + 4 qd + r, column
        // = step t, i.e. W's row fragment of key tile ib
#pragma unroll
        for (int ib = 0; ib < 4; ++ib)
          o.w[ib][lane] = mm16(*reinterpret_cast<const f32x4*>(&my.ah[(16 * ib + t) * kLs + 4 * qd]), Pt, zero);
        // U = (P A_ak) V per value tile. (P A_ak)^T = A_ak^T P^T in the
        // result layout is P A_ak's row fragment: lane (qd, t) holds
        // (P A_ak)[t][4 qd + r]
        (void)P;
        const f32x4 pak = mm16(col4(my.aak, kLg, t, qd), Pt, zero);
#pragma unroll
        for (int vb = 0; vb < 4; ++vb) o.u[vb][lane] = mm16(pak, V[vb], zero);
#pragma unroll
        for (int vb = 0; vb < 4; ++vb) V[vb] = col_frag4(bv, tstride, cn, t, vb, qd);
        // the next chunk's x rows, for the chain waves to turn into gamma_t
        if (cn != c) {
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) *reinterpret_cast<f32x4*>(&dx[s][dx_at(t, 4 * kk + qd)]) = X[kk];
        }
        lds_release();
        if (lane == 0) lds_store_flag(&flags.ready[s], c);
      }
    }
  } else {
    // ===================================================== chain wave: value tile jb
    // state: key tiles ib in the result layout (rows = key 16 ib + 4 qd + r,
    // column = value jcol)
    const int jb = wave, jcol = 16 * jb + t;
    f32x4 S[4];
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) {
      // s0 is [value][key]: register r holds key 16 ib + 4 qd + r of value jcol
      if (kHasS0)
        S[ib] = *reinterpret_cast<const f32x4*>(p.s0 + bh * (kHead * kHead) + jcol * kHead + 16 * ib + 4 * qd);
      else
        S[ib] = zero;
    }
    // the checkpoint after checkpoint group n, transposed ([key][value])
    auto store_ckpt = [&](int n) {
      float* const ck = p.ckpt + (bh * (T / p.C) + n) * (kHead * kHead);
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int r = 0; r < 4; ++r) ck[(16 * ib + 4 * qd + r) * kHead + jcol] = S[ib][r];
    };
    for (int c = 0; c < nchunks; ++c) {
      const int slot = c % kSlots;
      if (!wait_flag(&flags.ready[slot], c, p.spin_limit) && lane == 0) lds_store_flag(&flags.fault, 1);
      lds_acquire();
      const F32ChunkOps& o = ops[slot];
      f32x4 w[4], rh[4], ke[4], be[4], gl[4];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
        w[ib] = o.w[ib][lane];
        rh[ib] = o.rh[ib][lane];
        ke[ib] = *reinterpret_cast<const f32x4*>(&o.ke[(16 * ib + t) * kLs + 4 * qd]);
        be[ib] = *reinterpret_cast<const f32x4*>(&o.be[(16 * ib + t) * kLs + 4 * qd]);
        gl[ib] = *reinterpret_cast<const f32x4*>(&o.gl[16 * ib + 4 * qd]);
      }
      const f32x4 ark = o.ark[lane], arb = o.arb[lane], vcol = o.v[jb][lane], u = o.u[jb][lane];
      // gamma_t of chunk c + 4, keys 16 jb + 4 qd + r (a chunk past the end
      // works on stale rows that nobody reads: no branch in the products' block)
      float* const gx = &dx[slot][dx_at(t, 4 * jb + qd)];
      const f32x4 xv = *reinterpret_cast<const f32x4*>(gx);
      // every operand load is issued before the first product, so the loads'
      // latencies overlap instead of one wait per operand
      __builtin_amdgcn_sched_barrier(0);
      f32x4 gv;
#pragma unroll
      for (int r = 0; r < 4; ++r) gv[r] = gamma_of(xv[r]);

      f32x4 sa = u;
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) sa = mm16(w[ib], S[ib], sa);
      f32x4 y = zero;
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) y = mm16(rh[ib], S[ib], y);
      y = mm16(ark, vcol, y);
      y = mm16(arb, sa, y);
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
        f32x4 st = S[ib] * gl[ib];
        st = mm16(ke[ib], vcol, st);
        st = mm16(be[ib], sa, st);
        S[ib] = st;
      }
      *reinterpret_cast<f32x4*>(gx) = gv;
      // every operand has been used, so its load has completed (the wait costs
      // nothing here); the slot goes back to its prep wave
      __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
      lds_release();
      if (lane == 0) lds_store_flag(&flags.taken[slot][jb], c);
      // outputs: rows = steps 16 c + 4 qd + r, column = value jcol
      const int64_t cbase = tok0 + (int64_t)kL * c * tstride;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p.sa[cbase + (int64_t)(4 * qd + r) * tstride + jcol] = sa[r];
        Io<Tin>::put1(&p.y[cbase + (int64_t)(4 * qd + r) * tstride + jcol], y[r]);
      }
      if ((c + 1) % per_ckpt == 0) store_ckpt((c + 1) / per_ckpt - 1);
    }
    if (p.sT) {
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
        *reinterpret_cast<f32x4*>(p.sT + bh * (kHead * kHead) + jcol * kHead + 16 * ib + 4 * qd) = S[ib];
    }
  }

  // every wave ends here: if any wave gave up a wait, the whole (batch,
  // head)'s outputs are unreliable, so they are overwritten with NaN and the
  // event is counted for the host
  __syncthreads();
  if (lds_load_flag(&flags.fault)) {
    const float nan = __builtin_nanf("");
    for (int64_t i = tid; i < (int64_t)T * kHead; i += kBlock) {
      const int64_t off = tok0 + (i >> 6) * tstride + (i & 63);
      Io<Tin>::put1(&p.y[off], nan);
      p.sa[off] = nan;
    }
    float* const ck = p.ckpt + bh * (T / p.C) * (kHead * kHead);
    for (int64_t i = tid; i < (int64_t)(T / p.C) * kHead * kHead; i += kBlock) ck[i] = nan;
    if (p.sT)
      for (int i = tid; i < kHead * kHead; i += kBlock) p.sT[bh * (kHead * kHead) + i] = nan;
    if (tid == 0) atomicAdd(p.faults, 1u);
  }
}

// ------------------------------------------------------------------ backward
enum { I_X, I_R, I_K, I_V, I_A, I_B, I_DY, I_SA, I_COUNT };   // staged rows
enum { Y_YV, Y_YSA, Y_SAV, Y_SASA, Y_COUNT };                  // step products of the gradient
enum { O_DW, O_DR, O_DK, O_DV, O_DA, O_DB, O_COUNT };

struct F32BwdParams {
  const float* in[I_COUNT];   // [B,T,H,64] each (the removal_state last)
  const float* ckpt;          // [B,H,T/C,64(key),64(value)]
  const float* dsT;           // [B,H,64(value),64(key)] or null
  float* g[O_COUNT];          // gradients [B,T,H,64]
  float* ds0;                 // [B,H,64(value),64(key)] or null
  int T, H, C;
};

struct F32BwdLds {
  f32x4 sb[4][4][64];             // a chunk's start state S0, per key tile: [jj][lane]
  float raw[I_COUNT][kL * kLd];   // the chunk's rows
  float dec[D_COUNT][kL * kLd];   // decayed rows, [step][key]
  float gam[kL * kLd];            // gamma_t, [step][key]
  float gpv[kL * kLd];            // gamma_{t-1}
  float winv[kL * kLd];           // 1 / w~, [step][key]
  float g[G_COUNT][kL * kLg];     // A_ab, A_ak, A_rb, A_rk, [t][s]
  float pm[kL * kLg];             // P = (I - A_ab)^-1
  float by[Y_COUNT][kL * kLg];    // B_yv, B_ysa, B_sav, B_sasa, [t][s]
  float dsa[kL * kLd];            // dSA, [step][value]
  float ds[64 * kLd];             // the chunk-end state gradient dS, [value][key]
  float out[O_COUNT][kL * kLd];   // a chunk's gradients, [step][key or value]
  float fra[kL * kLd];            // r dr + a da, [step][key]
  float es0[64];                  // gamma_L sum_j S0 dS, per key
  float gl[64];                   // gamma_L
};

// One workgroup of 8 waves per (batch, head), chunks in reverse order. With
// dS the gradient of the chunk's end state, S0 its start state, and the
// chunk's products as in the forward (K- = K~ gamma_L, B- = B~ gamma_L):
//   dSA = P^T (B- dS^T + A_rb^T dY),  dV = K- dS^T + A_rk^T dY + A_ak^T dSA,
//   dS_prev = dS diag(gamma_L) + dY^T R^ + dSA^T A^ (carried to chunk c - 1),
//   dK = (B_yv R^ + B_sav A^ + (V dS) diag(gamma_L)) / gamma,
//   dB = (B_ysa R^ + B_sasa A^ + (SA dS) diag(gamma_L)) / gamma,
//   dR = gamma (dY S0 + B_yv^T K~ + B_ysa^T B~),
//   dA = gamma_{t-1} (dSA S0 + B_sav^T K~ + B_sasa^T B~),
// with B_yv[t][s] = v_t . dy_s (s >= t), B_ysa = sa_t . dy_s (s >= t),
// B_sav = v_t . dsa_s (s > t), B_sasa = sa_t . dsa_s (s > t). The log-decay
// gradient of step u is the suffix sum over t >= u of r dr + a da - k dk -
// b db, minus a_u da_u, plus the chunk-end term E = sum_t (K- o V dS + B- o
// SA dS) + gamma_L o sum_j (S0 o dS); dw = W_SCALE sigmoid (1 - sigmoid) of
// that.
//
// Waves 0-3 ("chain waves", value tile w and key tile w) carry dS and never
// store to memory; waves 4-7 ("key waves", key tile w - 4) issue every
// store. The key waves own a chunk's start state S0: a checkpoint, or where
// none holds it, the reference's reversal from the chunk's end state,
// spread over the phases in which the chain waves' products keep the
// matrix cores busy; they hand it to the chain waves through LDS. On this
// hardware one
// counter tracks a wave's loads and stores in issue order, so a wave that
// waits for a load also waits for every store it issued before it (and the
// compiler's wait at the top of a loop iteration counts the previous
// iteration's stores): kept apart, the chain waves' waits for the next
// chunk's rows do not wait for the gradients, and the key waves issue their
// loads after their stores, a whole chunk before they wait for them. Phases (barriers
// between):
//   stage the chunk's rows (loaded in the previous key stage); finish dw of
//           the previous chunk and store its gradients, read a checkpointed
//           S0 (key waves)
//   decays, decayed rows, gamma_t, gamma_{t-1}, 1 / w~
//   A_ab and P, A_ak, A_rb, A_rk (waves 0-3); B_yv, B_ysa (waves 4, 5);
//           reversal steps 15-11 (key waves)
//   dSA, dV (waves 0-3: value tile w), dS and dSA to LDS; reversal steps
//           10-5 (key waves)
//   dS_prev (waves 0-3); B_sav, B_sasa (waves 4, 5); reversal steps 4-0,
//           S0 to LDS (key waves)
//   key-indexed gradients of key tile w: dR, dA and their part of the decay
//           gradient (chain waves, S0 from LDS), dK, dB and theirs (key waves)
__global__ __launch_bounds__(kBlock, 1) void wkv7_bwd_f32_chunk_kernel(const F32BwdParams p) {
  __shared__ F32BwdLds L;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = tid >> 6;
  const int t = lane & 15, qd = lane >> 4;
  const int h = blockIdx.x, b = blockIdx.y, H = p.H, T = p.T;
  const int64_t bh = (int64_t)b * H + h;
  const int64_t tstride = (int64_t)H * kHead;
  const int64_t tok0 = ((int64_t)b * T * H + h) * kHead;
  const int nchunks = T / kL;
  const int q = p.C / kL;                           // 16-step chunks per checkpoint
  const bool chain = wave < 4;
  const int wq = wave & 3;
  const int jcol = 16 * wq + t;                     // chain waves: the lane's value
  const int ki = 16 * wq + t;                       // the lane's key in the key stage
  const int ctid = tid & 255;                       // thread index within its group of 4 waves
  const float* const ckbh = p.ckpt + bh * (T / p.C) * (kHead * kHead);

  // staging: 8 row tensors x 16 steps x 16 float4 = 2048 float4; the
  // chain waves load x, r, k, v and the key waves a, b, dy, sa, four per
  // thread, in the key stage of the chunk before; the key waves' stores
  // follow at the next stage, so the wait for the rows waits for no store.
  // (thread ctid: step row ctid / 16, 16-byte piece ctid % 16 of each
  // tensor; a uniform base per tensor and chunk, one 32-bit lane offset)
  f32x4 stg[4];
  const int vec0 = chain ? I_X : I_A;
  const int srow = ctid >> 4, sc4 = ctid & 15;
  const uint32_t soff = (uint32_t)srow * (uint32_t)tstride + 4 * sc4;
  auto fetch = [&](int c) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const float* const base = p.in[vec0 + m] + tok0 + (int64_t)kL * c * tstride;
      stg[m] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(base + soff));
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int m = 0; m < 4; ++m) *reinterpret_cast<f32x4*>(&L.raw[vec0 + m][srow * kLd + 4 * sc4]) = stg[m];
  };

  // chain waves: dS of the chunk end, rows = key 16 ib + 4 qd + r, column = value jcol
  f32x4 dS[4];
#pragma unroll
  for (int ib = 0; ib < 4; ++ib) {
    if (chain && p.dsT)
      dS[ib] = *reinterpret_cast<const f32x4*>(p.dsT + bh * (kHead * kHead) + jcol * kHead + 16 * ib + 4 * qd);
    else
      dS[ib] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // a state as the B operand of a contraction over values:
  // s[jj][r] = S[value 16 jj + 4 qd + r][key ki], i.e. checkpoint row ki
  auto load_ckpt = [&](int n, f32x4 (&s)[4]) {
    const float* const ck = ckbh + (int64_t)n * (kHead * kHead);
    const uint32_t off = (uint32_t)ki * kHead + 4 * qd;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) s[jj] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(ck + off + 16 * jj));
  };
  // key waves: Sr holds the start state of the chunk processed last, i.e.
  // the end state of the next one; a checkpoint replaces it, or the
  // reversal rebuilds the earlier start state from it in place; either is
  // handed to the chain waves through LDS (S0) for the key stage.
  f32x4 Sr[4], S0[4];
  if (!chain && nchunks > 0) load_ckpt(T / p.C - 1, Sr);   // the end state of the last chunk
  // the reference's reversal of steps hi .. lo (kernel.rs:239-246), in the
  // reference's operation order: S_{t-1} = (S_t - k v - b sa) * (1 / w~)
  // Each group's own state (the chain waves' dS, the key waves' Sr and dw
  // parts) is overwritten in the other group's branches, where it is
  // meaningless, so that its registers are free there.
  auto drop = [](f32x4 (&v)[4]) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) v[jj] = f32x4{0.f, 0.f, 0.f, 0.f};
  };
  auto reverse = [&](int hi, int lo) {
#pragma clang fp contract(off)
#pragma unroll 1
    for (int tt = hi; tt >= lo; --tt) {
      const float winv = L.winv[tt * kLd + ki];
      const float kv = L.raw[I_K][tt * kLd + ki], bv = L.raw[I_B][tt * kLd + ki];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const f32x4 vv = *reinterpret_cast<const f32x4*>(&L.raw[I_V][tt * kLd + 16 * jj + 4 * qd]);
        const f32x4 sv = *reinterpret_cast<const f32x4*>(&L.raw[I_SA][tt * kLd + 16 * jj + 4 * qd]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float t1 = kv * vv[r];
          const float t2 = Sr[jj][r] - t1;
          const float t3 = bv * sv[r];
          Sr[jj][r] = (t2 - t3) * winv;
        }
      }
    }
  };

  // key waves: the previous chunk's part of the decay gradient (k dk + b db,
  // the chunk-end term's K- and B- parts) and W_SCALE sigmoid (1 - sigmoid)
  // of the lane's steps, kept in registers (the chain waves overwrite the x
  // rows while the key waves finish it; the a rows are the key waves' own)
  f32x4 fkb = {0.f, 0.f, 0.f, 0.f}, sgk = fkb;
  float ekb = 0.f;
  auto finish_and_store = [&](int cc) {
    const f32x4 fra = col4(L.fra, kLd, ki, qd), da = col4(L.out[O_DA], kLd, ki, qd);
    const f32x4 akb = col4(L.raw[I_A], kLd, ki, qd);
    const float etot = rows_total(ekb) + L.es0[ki];
    const f32x4 f = fra - fkb;
    f32x4 suf;
    suf[3] = f[3];
    suf[2] = f[2] + suf[3];
    suf[1] = f[1] + suf[2];
    suf[0] = f[0] + suf[1];
    const float above = rows_after(suf[0], qd);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      L.out[O_DW][(4 * qd + r) * kLd + ki] = (suf[r] + above - akb[r] * da[r] + etot) * sgk[r];
    wave_lds_sync();
    // this wave's key (or value) columns 16 wq .. 16 wq + 15 of the six
    // gradient tiles, as 16-byte pieces: tile m, row l / 4, piece 4 wq + l % 4
    const int64_t cbase = tok0 + (int64_t)kL * cc * tstride;
    const int row = lane >> 2, c4 = 4 * wq + (lane & 3);
    const uint32_t off = (uint32_t)row * (uint32_t)tstride + 4 * c4;
#pragma unroll
    for (int m = 0; m < O_COUNT; ++m)
      __builtin_nontemporal_store(*reinterpret_cast<const f32x4*>(&L.out[m][row * kLd + 4 * c4]),
                                  reinterpret_cast<f32x4*>(p.g[m] + cbase + off));
  };

  if (nchunks > 0) fetch(nchunks - 1);
  for (int c = nchunks - 1; c >= 0; --c) {
    const bool from_ckpt = c > 0 && c % q == 0;
    if (chain) {
      stage();
    } else {
      // dw of chunk c + 1 needs the chain waves' part, written in its key
      // stage, and its a rows, which this stage replaces
      if (c < nchunks - 1) finish_and_store(c + 1);
      stage();
      // a checkpointed start state replaces the reversal (read after the
      // stores, waited for three phases later)
      if (from_ckpt) load_ckpt(c / q - 1, Sr);
    }
    lds_barrier();

    // ---- decays (wave w: keys 8 w + 2 qd (+1), step t)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int key = 8 * wave + 2 * qd + e;
      const float x = L.raw[I_X][t * kLd + key];
      const float wt = expf(kWScale * (1.0f / (1.0f + expf(-x))));
      const float gam = row_prod16(wt);
      const float gpv = row_prev16(gam);
      const float gin = 1.0f / gam;
      const float gL = row_last16(gam);
      const float kt = L.raw[I_K][t * kLd + key] * gin, bt = L.raw[I_B][t * kLd + key] * gin;
      L.dec[D_AH][t * kLd + key] = L.raw[I_A][t * kLd + key] * gpv;
      L.dec[D_RH][t * kLd + key] = L.raw[I_R][t * kLd + key] * gam;
      L.dec[D_KT][t * kLd + key] = kt;
      L.dec[D_BT][t * kLd + key] = bt;
      L.dec[D_KE][t * kLd + key] = kt * gL;
      L.dec[D_BE][t * kLd + key] = bt * gL;
      L.gam[t * kLd + key] = gam;
      L.gpv[t * kLd + key] = gpv;
      L.winv[t * kLd + key] = 1.0f / wt;
      if (t == 0) L.gl[key] = gL;
    }
    lds_barrier();

    // ---- step products: A_ab and P (wave 0), A_ak, A_rb, A_rk (1-3);
    // B_yv, B_ysa (4, 5)
    if (chain) {
      drop(Sr);
      const int xa = wave < 2 ? D_AH : D_RH;
      const int zb = (wave & 1) ? D_KT : D_BT;
      f32x4 d = gram64(L.dec[xa], L.dec[zb], t, qd);
      const int strict = wave < 2 ? 1 : 0;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        d[r] = (4 * qd + r - t >= strict) ? d[r] : 0.f;
        L.g[wave][(4 * qd + r) * kLg + t] = d[r];
      }
      if (wave == 0) {
        wave_lds_sync();
        const f32x4 dt = *reinterpret_cast<const f32x4*>(&L.g[G_AB][t * kLg + 4 * qd]);
        f32x4 P, Pt;
        unit_lower_inverse_f32(d, dt, t, qd, P, Pt);
#pragma unroll
        for (int r = 0; r < 4; ++r) L.pm[(4 * qd + r) * kLg + t] = P[r];
      }
    } else {
      drop(dS);
      if (wq < 2) {
        f32x4 d = gram64(L.raw[wq == 0 ? I_V : I_SA], L.raw[I_DY], t, qd);   // [t'][s] = x_t' . dy_s
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          d[r] = (t - (4 * qd + r) >= 0) ? d[r] : 0.f;                        // s >= t'
          L.by[wq][(4 * qd + r) * kLg + t] = d[r];
        }
      }
      if (!from_ckpt) reverse(kL - 1, 11);
    }
    lds_barrier();

    // ---- dSA and dV (chain waves, value tile wq)
    f32x4 dsa = {0.f, 0.f, 0.f, 0.f};
    f32x4 dycol = {0.f, 0.f, 0.f, 0.f};
    if (chain) {
      drop(Sr);
      dycol = col4(L.raw[I_DY], kLd, jcol, qd);
      f32x4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) x = mm16(row4(L.dec[D_BE], kLd, t, 16 * ib, qd), dS[ib], x);
      x = mm16(col4(L.g[G_RB], kLg, t, qd), dycol, x);
      dsa = mm16(col4(L.pm, kLg, t, qd), x, dsa);
      f32x4 dv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) dv = mm16(row4(L.dec[D_KE], kLd, t, 16 * ib, qd), dS[ib], dv);
      dv = mm16(col4(L.g[G_RK], kLg, t, qd), dycol, dv);
      dv = mm16(col4(L.g[G_AK], kLg, t, qd), dsa, dv);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        L.dsa[(4 * qd + r) * kLd + jcol] = dsa[r];
        L.out[O_DV][(4 * qd + r) * kLd + jcol] = dv[r];
      }
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) *reinterpret_cast<f32x4*>(&L.ds[jcol * kLd + 16 * ib + 4 * qd]) = dS[ib];
    } else {
      drop(dS);
      if (!from_ckpt) reverse(10, 5);
    }
    lds_barrier();

    // ---- dS_prev (chain waves); B_sav, B_sasa (waves 4, 5)
    if (chain) {
      drop(Sr);
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
        const f32x4 gl = *reinterpret_cast<const f32x4*>(&L.gl[16 * ib + 4 * qd]);
        f32x4 s = dS[ib] * gl;
        s = mm16(col4(L.dec[D_RH], kLd, 16 * ib + t, qd), dycol, s);
        s = mm16(col4(L.dec[D_AH], kLd, 16 * ib + t, qd), dsa, s);
        dS[ib] = s;
      }
    } else {
      drop(dS);
      if (wq < 2) {
        f32x4 d = gram64(L.raw[wq == 0 ? I_V : I_SA], L.dsa, t, qd);           // [t'][s] = x_t' . dsa_s
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          d[r] = (t - (4 * qd + r) > 0) ? d[r] : 0.f;                          // s > t'
          L.by[Y_SAV + wq][(4 * qd + r) * kLg + t] = d[r];
        }
      }
      if (!from_ckpt) reverse(4, 0);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) L.sb[wq][jj][lane] = Sr[jj];
    }
    lds_barrier();

    // ---- key-indexed gradients of key tile wq: rows = step 4 qd + r,
    // column = key ki. The next chunk's rows are loaded first (their
    // registers are free from here to the next stage).
    if (c > 0) fetch(c - 1);
    const float gl = L.gl[ki];
    if (chain) {
      drop(Sr);
      fkb = sgk = f32x4{0.f, 0.f, 0.f, 0.f};
      ekb = 0.f;
      // dR, dA and r dr + a da; the chunk-end term's gamma_L sum_j S0 o dS
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) S0[jj] = L.sb[wq][jj][lane];
      f32x4 dr = {0.f, 0.f, 0.f, 0.f}, da = dr;
      float so = 0.f;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        dr = mm16(row4(L.raw[I_DY], kLd, t, 16 * jj, qd), S0[jj], dr);
        da = mm16(row4(L.dsa, kLd, t, 16 * jj, qd), S0[jj], da);
        const f32x4 dsc = col4(L.ds + 16 * jj * kLd, kLd, ki, qd);           // dS[16 jj + 4 qd + r][ki]
#pragma unroll
        for (int r = 0; r < 4; ++r) so += S0[jj][r] * dsc[r];
      }
      const f32x4 kt = col4(L.dec[D_KT], kLd, ki, qd), bt = col4(L.dec[D_BT], kLd, ki, qd);
      dr = mm16(col4(L.by[Y_YV], kLg, t, qd), kt, dr);
      dr = mm16(col4(L.by[Y_YSA], kLg, t, qd), bt, dr);
      da = mm16(col4(L.by[Y_SAV], kLg, t, qd), kt, da);
      da = mm16(col4(L.by[Y_SASA], kLg, t, qd), bt, da);
      const f32x4 gam = col4(L.gam, kLd, ki, qd), gpv = col4(L.gpv, kLd, ki, qd);
      const f32x4 rr = col4(L.raw[I_R], kLd, ki, qd), aa = col4(L.raw[I_A], kLd, ki, qd);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        dr[r] = dr[r] * gam[r];
        da[r] = da[r] * gpv[r];
        L.out[O_DR][(4 * qd + r) * kLd + ki] = dr[r];
        L.out[O_DA][(4 * qd + r) * kLd + ki] = da[r];
        L.fra[(4 * qd + r) * kLd + ki] = rr[r] * dr[r] + aa[r] * da[r];
      }
      const float st = rows_total(so);
      if (qd == 0) L.es0[ki] = gl * st;
    } else {
      drop(dS);
      // dK, dB and k dk + b db; the chunk-end term's K- and B- parts
      f32x4 dke = {0.f, 0.f, 0.f, 0.f}, dbe = dke;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const f32x4 dsc = col4(L.ds + 16 * jj * kLd, kLd, ki, qd);
        dke = mm16(row4(L.raw[I_V], kLd, t, 16 * jj, qd), dsc, dke);
        dbe = mm16(row4(L.raw[I_SA], kLd, t, 16 * jj, qd), dsc, dbe);
      }
      const f32x4 rh = col4(L.dec[D_RH], kLd, ki, qd), ah = col4(L.dec[D_AH], kLd, ki, qd);
      f32x4 dk = dke * gl, db = dbe * gl;
      dk = mm16(row4(L.by[Y_YV], kLg, t, 0, qd), rh, dk);
      dk = mm16(row4(L.by[Y_SAV], kLg, t, 0, qd), ah, dk);
      db = mm16(row4(L.by[Y_YSA], kLg, t, 0, qd), rh, db);
      db = mm16(row4(L.by[Y_SASA], kLg, t, 0, qd), ah, db);
      const f32x4 gam = col4(L.gam, kLd, ki, qd);
      const f32x4 ke = col4(L.dec[D_KE], kLd, ki, qd), be = col4(L.dec[D_BE], kLd, ki, qd);
      const f32x4 kk = col4(L.raw[I_K], kLd, ki, qd), bb = col4(L.raw[I_B], kLd, ki, qd);
      const f32x4 xx = col4(L.raw[I_X], kLd, ki, qd);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float sg = 1.0f / (1.0f + expf(-xx[r]));
        sgk[r] = kWScale * sg * (1.0f - sg);
      }
      ekb = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        ekb += ke[r] * dke[r] + be[r] * dbe[r];
        dk[r] = dk[r] / gam[r];
        db[r] = db[r] / gam[r];
        L.out[O_DK][(4 * qd + r) * kLd + ki] = dk[r];
        L.out[O_DB][(4 * qd + r) * kLd + ki] = db[r];
        fkb[r] = kk[r] * dk[r] + bb[r] * db[r];
      }
    }
    lds_barrier();
  }
  if (!chain && nchunks > 0) finish_and_store(0);
  if (chain && p.ds0) {
#pragma unroll
    for (int ib = 0; ib < 4; ++ib)
      *reinterpret_cast<f32x4*>(p.ds0 + bh * (kHead * kHead) + jcol * kHead + 16 * ib + 4 * qd) = dS[ib];
  }
}

}  // namespace

// fp32 operands at chunk_len 16 and 32, bf16 operands at 32 (at 16 the
// split-bf16 chunked forward runs). Past 32 the step forward runs: the
// backward rebuilds the start states between checkpoints by the reference's
// reversal, which multiplies a checkpoint's deviation by about 1.35 per
// step, and this kernel's checkpoints (chunked products of the decays) sit
// 1.7e-7 from the reference order's where the step forward's sit 5-7e-8.
// Measured against exact gradients, at chunk_len 48 and 64 that left dw,
// dr, da 2-3 times further off than the reference algorithm itself, while
// from the step forward's checkpoints they match its accuracy; at 32 both
// stay within 1.2 times of it (and within bf16 rounding for bf16 operands).
bool chunk_f32_forward_supported(const ForwardDesc& d) {
  const bool io = d.dtype == Dtype::F32 || (d.dtype == Dtype::BF16 && d.C > kL);
  return io && d.C % kL == 0 && d.C <= 2 * kL && d.T % d.C == 0;
}

template <typename Tin>
static hipError_t launch_fwd_f32(const ForwardDesc& d, hipStream_t stream) {
  F32FwdParams<Tin> p;
  p.in[R_X] = static_cast<const Tin*>(d.w);
  p.in[R_R] = static_cast<const Tin*>(d.r);
  p.in[R_K] = static_cast<const Tin*>(d.k);
  p.in[R_V] = static_cast<const Tin*>(d.v);
  p.in[R_A] = static_cast<const Tin*>(d.a);
  p.in[R_B] = static_cast<const Tin*>(d.b);
  p.s0 = d.s0;
  p.ckpt = d.ckpt;
  p.sa = d.sa;
  p.y = static_cast<Tin*>(d.y);
  p.sT = d.sT;
  p.T = d.T;
  p.H = d.H;
  p.C = d.C;
  p.spin_limit = d.kc.spin_limit ? d.kc.spin_limit : kSpinLimit;
  // the counter lives in the bf16 forward's code object; its address is
  // looked up on the current device at every launch (a host-side lookup, no
  // stream work, so captured launches replay it as they are)
  hipError_t e = handover_fault_counter(&p.faults);
  if (e != hipSuccess) return e;
  const dim3 grid(d.H, d.B, 1), block(kBlock, 1, 1);
  if (d.s0)
    hipLaunchKernelGGL((wkv7_fwd_f32_chunk_kernel<Tin, true>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((wkv7_fwd_f32_chunk_kernel<Tin, false>), grid, block, 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_forward_chunked_f32(const ForwardDesc& d, hipStream_t stream) {
  return d.dtype == Dtype::BF16 ? launch_fwd_f32<bf16_t>(d, stream) : launch_fwd_f32<float>(d, stream);
}

}  // namespace wkv7

namespace wkv7 {

bool chunk_f32_backward_supported(const BackwardDesc& d) {
  return d.dtype == Dtype::F32 && d.C % kL == 0 && d.T % d.C == 0 && d.T > 0;
}

// Between checkpoints the chunked backward rebuilds each 16-step chunk's
// start state by the reference's reversal, on its key waves, a pass per
// rebuilt chunk that the step kernels (which reverse every step anyway) do
// not pay: one of every two chunks at chunk_len 32, three of four at 64.
// Backward alone, one box, fp32: at chunk_len 32 the chunked kernel is as
// fast or faster from 64 (batch, head) pairs up (2% at 128, 10% at 256) and
// 1-3% slower at 8-16 pairs; at chunk_len 64 it is 7-10% slower at 8-128
// pairs and 0.5-3% faster at 256 (one workgroup per CU). At chunk_len 16
// every chunk starts at a checkpoint and it is 15-26% faster throughout.
bool chunk_f32_backward_preferred(const BackwardDesc& d) {
  return d.C <= 2 * kL || (int64_t)d.B * d.H >= 256;
}

hipError_t launch_backward_chunked_f32(const BackwardDesc& d, hipStream_t stream) {
  F32BwdParams p;
  p.in[I_X] = static_cast<const float*>(d.w);
  p.in[I_R] = static_cast<const float*>(d.r);
  p.in[I_K] = static_cast<const float*>(d.k);
  p.in[I_V] = static_cast<const float*>(d.v);
  p.in[I_A] = static_cast<const float*>(d.a);
  p.in[I_B] = static_cast<const float*>(d.b);
  p.in[I_DY] = static_cast<const float*>(d.dy);
  p.in[I_SA] = d.sa;
  p.ckpt = d.ckpt;
  p.dsT = d.dsT;
  p.g[O_DW] = static_cast<float*>(d.dw);
  p.g[O_DR] = static_cast<float*>(d.dr);
  p.g[O_DK] = static_cast<float*>(d.dk);
  p.g[O_DV] = static_cast<float*>(d.dv);
  p.g[O_DA] = static_cast<float*>(d.da);
  p.g[O_DB] = static_cast<float*>(d.db);
  p.ds0 = d.ds0;
  p.T = d.T;
  p.H = d.H;
  p.C = d.C;
  hipLaunchKernelGGL(wkv7_bwd_f32_chunk_kernel, dim3(d.H, d.B, 1), dim3(kBlock, 1, 1), 0, stream, p);
  return hipGetLastError();
}

}  // namespace wkv7
