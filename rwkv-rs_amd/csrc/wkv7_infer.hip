// WKV7 slot-mapped inference (decode / prefill) for gfx950, forward only.
//
// Semantics: /root/reference/crates/rwkv-nn/src/kernels/wkv7_infer/kernel.rs:15-114
// (wkv7_infer_forward_kernel). Active row b works on state slot batch_ids[b]
// of a [full_batch, H, 64, 64] state buffer, read and written in place
// (kernel.rs:27-42, 103-113). A step whose context_mask entry is 0 writes
// y = 0 and leaves the state untouched (kernel.rs:57-62). With use_dither
// (bf16 state only) the decay gets deterministic_dither(elapsed_t[slot] +
// valid_t) added, where valid_t counts the unmasked steps of this call before
// the current one (kernel.rs:8-13, 73-77).
//
// Two state element types, as the reference's kernel is instantiated:
// - fp32 state (wkv7_infer_kernel): the reference at F = f32, which runs
//   without the dither (host.rs:157); bf16 operands are carried as their
//   exact fp32 values.
// - bf16 state (wkv7_infer_bf16_kernel): the reference at F = bf16. The
//   state, the staged operands and every product and sum are bf16: the decay
//   is formed in fp32, gets the dither, and is rounded to bf16 once
//   (kernel.rs:71-78); the removal-state sum, the state update and the output
//   sum round each operation to bf16 in the kernel's order (kernel.rs:81-98),
//   summing over the key index left to right.
//
// Design of the fp32-state kernel: the forward kernel's thread layout and
// per-step arithmetic (one workgroup per (active row, head), a 2x4 state
// block per thread in VGPRs, operands from LDS). At T = 1 it is bound by the
// 16 KiB state read and 16 KiB state write per (row, head): every thread
// moves two 16-byte rows each way, and the grid has Ba*H workgroups.
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
  Tin* y;
  int T, H, full_batch;
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
  const int64_t tstride = (int64_t)p.H * kHead;
  const int64_t tok0 = ((int64_t)bi * T * p.H + h) * kHead;

  float* st = p.state + (slot * p.H + h) * (kHead * kHead) + 4 * L;
  float So[4], St[4];   // own and other row
  {
    // The state is read and written once per call with the non-temporal
    // hint: a serving loop decodes every layer in turn, so a layer's state is
    // not in the caches when its next step comes (measured at config[3] with
    // the state read from HBM: 65.7 -> 60.1 us; with one state buffer reused
    // from the caches step after step the hint costs 50.6 -> 57.5 us)
    typedef float nt4 __attribute__((ext_vector_type(4)));
    const nt4 y0 = __builtin_nontemporal_load(reinterpret_cast<const nt4*>(st + ro * kHead));
    const nt4 y1 = __builtin_nontemporal_load(reinterpret_cast<const nt4*>(st + rt * kHead));
    const float4 x0 = make_float4(y0.x, y0.y, y0.z, y0.w), x1 = make_float4(y1.x, y1.y, y1.z, y1.w);
    So[0] = x0.x; So[1] = x0.y; So[2] = x0.z; So[3] = x0.w;
    St[0] = x1.x; St[1] = x1.y; St[2] = x1.z; St[3] = x1.w;
  }

  typedef Io<Tin> io;
  typename io::raw pre[V_COUNT];
  bool pre_live = true;

  auto gload = [&](int t0) {
    const int t = t0 + sl;
    if (stager && t < T) {
      pre_live = !p.mask || mask_on<Tin>(p.mask, (int64_t)bi * T + t);
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
      if (pp == 0) live[buf][sl] = pre_live ? 1 : 0;
    }
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

  typedef float nt4s __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store(nt4s{So[0], So[1], So[2], So[3]}, reinterpret_cast<nt4s*>(st + ro * kHead));
  __builtin_nontemporal_store(nt4s{St[0], St[1], St[2], St[3]}, reinterpret_cast<nt4s*>(st + rt * kHead));
}

// ------------------------------------------------------------ bf16 state
// One wave per (active row, head); lane j owns value row j of the state, so
// each row's sums over the key index run left to right inside one lane, as
// the reference's thread j does (kernel.rs:81-96). The row is held as 32
// registers of bf16 pairs, as stored, and never widened. The step's
// key-indexed operands (the rounded decay, a, b, k, r) go through LDS and are
// read back as broadcasts; lane j keeps its own v_j. The step is mostly VALU
// work (64 x 64 elements of one (row, head) on
// one wave, a rounding after every operation): each product of two bf16
// values is one bf16 dot product, each "round two values, add them" one
// packed conversion and one bf16 dot product (see the blocks below), and the
// two new state values of a key pair are rounded by one packed conversion. The
// 8 KiB state moves between HBM and the lanes' rows
// through LDS, with coalesced 16-byte accesses on the HBM side and each row's
// 16-byte pieces rotated by row + row / 8 so that neither the row-per-lane
// reads nor the contiguous writes conflict on LDS banks.
struct InferBf16Params {
  const bf16_t *w, *r, *k, *v, *a, *b;
  const int32_t* batch_ids;
  bf16_t* state;
  const bf16_t* mask;
  const int32_t* elapsed_t;
  bf16_t* y;
  int T, H, full_batch, use_dither;
};

__device__ __forceinline__ int rot_piece(int row, int q) { return row * 8 + ((q + row + (row >> 3)) & 7); }

// The step's arithmetic is built on v_dot2_f32_bf16 in its VOP3P form,
// a.b + 0 with a zero constant accumulator: the compiler emits only the VOP2
// v_dot2c_f32_bf16, whose accumulator is its destination, and so needs a
// move of zero before every use (256 per step here). The VOP3P form is
// reachable through inline assembly only, where the compiler's hazard
// recognizer cannot see it. The kernel has no matrix-core instructions. Two
// uses:
// - a product of two bf16 values, exact in fp32, is one dot product of the
//   state pair with an operand word that holds the key's value in the half
//   of the key's parity and zero in the other (no widening of the state);
// - the reference's rounded sum rb(x + p) of two fp32 values is the dot
//   product of their packed bf16 roundings with (1, 1), whose bf16 rounding
//   is that of the fp32 addition (add_rb in wkv7_device.hpp, checked on the
//   device by tests/test_gpu_selftest.py).
// A DOT result may be read by another VALU instruction three wait states
// after it is written (what the compiler keeps after v_dot2 on gfx950: an
// s_nop 2 directly after it, fewer nops when other instructions come
// between), and the blocks keep the same spacing before a non-DOT
// instruction overwrites a DOT result. Each block below interleaves
// independent chains (the keys of a group, the next group's products, the
// previous group's terms of the y sum) so that those slots hold work instead
// of nops, and ends with s_nop 2, so code after it may read or overwrite any
// of its results. The order of every rounded operation of one key is the
// reference's.
constexpr uint32_t kOnes = 0x3f803f80u;   // bf16 (1, 1)

// the rounded sums of the sa chain for four keys (products p, formed by the
// block before), with the next four keys' products formed in the chain's
// wait slots
template <bool kNext>
__device__ __forceinline__ void sa_four(const float (&p)[4], uint32_t s01, uint32_t s23, uint4 a,
                                        float (&pn)[4], float& z) {
  uint32_t t;
  if constexpr (kNext) {
    asm("v_cvt_pk_bf16_f32 %[t], %[z], %[p0]\n\t"
        "v_dot2_f32_bf16 %[z], %[t], %[one], 0\n\t"
        "v_dot2_f32_bf16 %[n0], %[s01], %[ax], 0\n\t"
        "v_dot2_f32_bf16 %[n1], %[s01], %[ay], 0\n\t"
        "s_nop 0\n\t"
        "v_cvt_pk_bf16_f32 %[t], %[z], %[p1]\n\t"
        "v_dot2_f32_bf16 %[z], %[t], %[one], 0\n\t"
        "v_dot2_f32_bf16 %[n2], %[s23], %[az], 0\n\t"
        "v_dot2_f32_bf16 %[n3], %[s23], %[aw], 0\n\t"
        "s_nop 0\n\t"
        "v_cvt_pk_bf16_f32 %[t], %[z], %[p2]\n\t"
        "v_dot2_f32_bf16 %[z], %[t], %[one], 0\n\t"
        "s_nop 2\n\t"
        "v_cvt_pk_bf16_f32 %[t], %[z], %[p3]\n\t"
        "v_dot2_f32_bf16 %[z], %[t], %[one], 0\n\t"
        "s_nop 2"
        : [n0] "=&v"(pn[0]), [n1] "=&v"(pn[1]), [n2] "=&v"(pn[2]), [n3] "=&v"(pn[3]), [t] "=&v"(t),
          [z] "+v"(z)
        : [p0] "v"(p[0]), [p1] "v"(p[1]), [p2] "v"(p[2]), [p3] "v"(p[3]), [s01] "v"(s01), [s23] "v"(s23),
          [ax] "v"(a.x), [ay] "v"(a.y), [az] "v"(a.z), [aw] "v"(a.w), [one] "v"(kOnes));
  } else {
    asm("v_cvt_pk_bf16_f32 %[t], %[z], %[p0]\n\t"
        "v_dot2_f32_bf16 %[z], %[t], %[one], 0\n\t"
        "s_nop 2\n\t"
        "v_cvt_pk_bf16_f32 %[t], %[z], %[p1]\n\t"
        "v_dot2_f32_bf16 %[z], %[t], %[one], 0\n\t"
        "s_nop 2\n\t"
        "v_cvt_pk_bf16_f32 %[t], %[z], %[p2]\n\t"
        "v_dot2_f32_bf16 %[z], %[t], %[one], 0\n\t"
        "s_nop 2\n\t"
        "v_cvt_pk_bf16_f32 %[t], %[z], %[p3]\n\t"
        "v_dot2_f32_bf16 %[z], %[t], %[one], 0\n\t"
        "s_nop 2"
        : [t] "=&v"(t), [z] "+v"(z)
        : [p0] "v"(p[0]), [p1] "v"(p[1]), [p2] "v"(p[2]), [p3] "v"(p[3]), [one] "v"(kOnes));
  }
}
// the products of the first four keys
__device__ __forceinline__ void sa_products(uint32_t s01, uint32_t s23, uint4 a, float (&p)[4]) {
  asm("v_dot2_f32_bf16 %[p0], %[s01], %[ax], 0\n\t"
      "v_dot2_f32_bf16 %[p1], %[s01], %[ay], 0\n\t"
      "v_dot2_f32_bf16 %[p2], %[s23], %[az], 0\n\t"
      "v_dot2_f32_bf16 %[p3], %[s23], %[aw], 0\n\t"
      "s_nop 2"
      : [p0] "=&v"(p[0]), [p1] "=&v"(p[1]), [p2] "=&v"(p[2]), [p3] "=&v"(p[3])
      : [s01] "v"(s01), [s23] "v"(s23), [ax] "v"(a.x), [ay] "v"(a.y), [az] "v"(a.z), [aw] "v"(a.w));
}
// four keys (two state pairs A and B) of the update and their four products
// with r (yn); kLinks: the four terms of the y sum left by the block before
// (yp) are added in between, their chain filling the update's wait slots
template <bool kLinks>
__device__ __forceinline__ void update_four(uint32_t& pa, uint32_t& pb, uint4 w, const float (&sb)[4],
                                            const float (&kv)[4], uint4 r, const float (&yp)[4],
                                            float (&yn)[4], float& zy) {
  float a0, a1, b0, b1;
  uint32_t ta0, ta1, tb0, tb1, t;
  if constexpr (kLinks) {
    asm("v_dot2_f32_bf16 %[a0], %[pa], %[w0], 0\n\t"
        "v_dot2_f32_bf16 %[a1], %[pa], %[w1], 0\n\t"
        "v_cvt_pk_bf16_f32 %[t], %[zy], %[yp0]\n\t"
        "v_dot2_f32_bf16 %[zy], %[t], %[one], 0\n\t"
        "v_dot2_f32_bf16 %[b0], %[pb], %[w2], 0\n\t"
        "v_dot2_f32_bf16 %[b1], %[pb], %[w3], 0\n\t"
        "v_cvt_pk_bf16_f32 %[ta0], %[a0], %[sb0]\n\t"
        "v_cvt_pk_bf16_f32 %[t], %[zy], %[yp1]\n\t"
        "v_dot2_f32_bf16 %[zy], %[t], %[one], 0\n\t"
        "v_cvt_pk_bf16_f32 %[ta1], %[a1], %[sb1]\n\t"
        "v_cvt_pk_bf16_f32 %[tb0], %[b0], %[sb2]\n\t"
        "v_cvt_pk_bf16_f32 %[tb1], %[b1], %[sb3]\n\t"
        "v_cvt_pk_bf16_f32 %[t], %[zy], %[yp2]\n\t"
        "v_dot2_f32_bf16 %[zy], %[t], %[one], 0\n\t"
        "v_dot2_f32_bf16 %[a0], %[ta0], %[one], 0\n\t"
        "v_dot2_f32_bf16 %[a1], %[ta1], %[one], 0\n\t"
        "v_dot2_f32_bf16 %[b0], %[tb0], %[one], 0\n\t"
        "v_cvt_pk_bf16_f32 %[t], %[zy], %[yp3]\n\t"
        "v_dot2_f32_bf16 %[zy], %[t], %[one], 0\n\t"
        "v_dot2_f32_bf16 %[b1], %[tb1], %[one], 0\n\t"
        "v_cvt_pk_bf16_f32 %[ta0], %[a0], %[kv0]\n\t"
        "v_cvt_pk_bf16_f32 %[ta1], %[a1], %[kv1]\n\t"
        "v_cvt_pk_bf16_f32 %[tb0], %[b0], %[kv2]\n\t"
        "v_cvt_pk_bf16_f32 %[tb1], %[b1], %[kv3]\n\t"
        "v_dot2_f32_bf16 %[a0], %[ta0], %[one], 0\n\t"
        "v_dot2_f32_bf16 %[a1], %[ta1], %[one], 0\n\t"
        "v_dot2_f32_bf16 %[b0], %[tb0], %[one], 0\n\t"
        "v_dot2_f32_bf16 %[b1], %[tb1], %[one], 0\n\t"
        "s_nop 0\n\t"
        "v_cvt_pk_bf16_f32 %[pa], %[a0], %[a1]\n\t"
        "v_dot2_f32_bf16 %[y0], %[pa], %[r0], 0\n\t"
        "v_cvt_pk_bf16_f32 %[pb], %[b0], %[b1]\n\t"
        "v_dot2_f32_bf16 %[y1], %[pa], %[r1], 0\n\t"
        "v_dot2_f32_bf16 %[y2], %[pb], %[r2], 0\n\t"
        "v_dot2_f32_bf16 %[y3], %[pb], %[r3], 0\n\t"
        "s_nop 2"
        : [a0] "=&v"(a0), [a1] "=&v"(a1), [b0] "=&v"(b0), [b1] "=&v"(b1), [ta0] "=&v"(ta0),
          [ta1] "=&v"(ta1), [tb0] "=&v"(tb0), [tb1] "=&v"(tb1), [t] "=&v"(t), [y0] "=&v"(yn[0]),
          [y1] "=&v"(yn[1]), [y2] "=&v"(yn[2]), [y3] "=&v"(yn[3]), [pa] "+v"(pa), [pb] "+v"(pb),
          [zy] "+v"(zy)
        : [w0] "v"(w.x), [w1] "v"(w.y), [w2] "v"(w.z), [w3] "v"(w.w), [sb0] "v"(sb[0]), [sb1] "v"(sb[1]),
          [sb2] "v"(sb[2]), [sb3] "v"(sb[3]), [kv0] "v"(kv[0]), [kv1] "v"(kv[1]), [kv2] "v"(kv[2]),
          [kv3] "v"(kv[3]), [r0] "v"(r.x), [r1] "v"(r.y), [r2] "v"(r.z), [r3] "v"(r.w),
          [yp0] "v"(yp[0]), [yp1] "v"(yp[1]), [yp2] "v"(yp[2]), [yp3] "v"(yp[3]), [one] "v"(kOnes));
  } else {
    asm("v_dot2_f32_bf16 %[a0], %[pa], %[w0], 0\n\t"
        "v_dot2_f32_bf16 %[a1], %[pa], %[w1], 0\n\t"
        "v_dot2_f32_bf16 %[b0], %[pb], %[w2], 0\n\t"
        "v_dot2_f32_bf16 %[b1], %[pb], %[w3], 0\n\t"
        "v_cvt_pk_bf16_f32 %[ta0], %[a0], %[sb0]\n\t"
        "v_cvt_pk_bf16_f32 %[ta1], %[a1], %[sb1]\n\t"
        "v_cvt_pk_bf16_f32 %[tb0], %[b0], %[sb2]\n\t"
        "v_cvt_pk_bf16_f32 %[tb1], %[b1], %[sb3]\n\t"
        "v_dot2_f32_bf16 %[a0], %[ta0], %[one], 0\n\t"
        "v_dot2_f32_bf16 %[a1], %[ta1], %[one], 0\n\t"
        "v_dot2_f32_bf16 %[b0], %[tb0], %[one], 0\n\t"
        "v_dot2_f32_bf16 %[b1], %[tb1], %[one], 0\n\t"
        "v_cvt_pk_bf16_f32 %[ta0], %[a0], %[kv0]\n\t"
        "v_cvt_pk_bf16_f32 %[ta1], %[a1], %[kv1]\n\t"
        "v_cvt_pk_bf16_f32 %[tb0], %[b0], %[kv2]\n\t"
        "v_cvt_pk_bf16_f32 %[tb1], %[b1], %[kv3]\n\t"
        "v_dot2_f32_bf16 %[a0], %[ta0], %[one], 0\n\t"
        "v_dot2_f32_bf16 %[a1], %[ta1], %[one], 0\n\t"
        "v_dot2_f32_bf16 %[b0], %[tb0], %[one], 0\n\t"
        "v_dot2_f32_bf16 %[b1], %[tb1], %[one], 0\n\t"
        "s_nop 0\n\t"
        "v_cvt_pk_bf16_f32 %[pa], %[a0], %[a1]\n\t"
        "v_dot2_f32_bf16 %[y0], %[pa], %[r0], 0\n\t"
        "v_cvt_pk_bf16_f32 %[pb], %[b0], %[b1]\n\t"
        "v_dot2_f32_bf16 %[y1], %[pa], %[r1], 0\n\t"
        "v_dot2_f32_bf16 %[y2], %[pb], %[r2], 0\n\t"
        "v_dot2_f32_bf16 %[y3], %[pb], %[r3], 0\n\t"
        "s_nop 2"
        : [a0] "=&v"(a0), [a1] "=&v"(a1), [b0] "=&v"(b0), [b1] "=&v"(b1), [ta0] "=&v"(ta0),
          [ta1] "=&v"(ta1), [tb0] "=&v"(tb0), [tb1] "=&v"(tb1), [y0] "=&v"(yn[0]), [y1] "=&v"(yn[1]),
          [y2] "=&v"(yn[2]), [y3] "=&v"(yn[3]), [pa] "+v"(pa), [pb] "+v"(pb)
        : [w0] "v"(w.x), [w1] "v"(w.y), [w2] "v"(w.z), [w3] "v"(w.w), [sb0] "v"(sb[0]), [sb1] "v"(sb[1]),
          [sb2] "v"(sb[2]), [sb3] "v"(sb[3]), [kv0] "v"(kv[0]), [kv1] "v"(kv[1]), [kv2] "v"(kv[2]),
          [kv3] "v"(kv[3]), [r0] "v"(r.x), [r1] "v"(r.y), [r2] "v"(r.z), [r3] "v"(r.w), [one] "v"(kOnes));
    (void)t;
  }
}
// the last four terms of the y sum
__device__ __forceinline__ void y_links(const float (&yp)[4], float& zy) {
  uint32_t t;
  asm("v_cvt_pk_bf16_f32 %[t], %[zy], %[yp0]\n\t"
      "v_dot2_f32_bf16 %[zy], %[t], %[one], 0\n\t"
      "s_nop 2\n\t"
      "v_cvt_pk_bf16_f32 %[t], %[zy], %[yp1]\n\t"
      "v_dot2_f32_bf16 %[zy], %[t], %[one], 0\n\t"
      "s_nop 2\n\t"
      "v_cvt_pk_bf16_f32 %[t], %[zy], %[yp2]\n\t"
      "v_dot2_f32_bf16 %[zy], %[t], %[one], 0\n\t"
      "s_nop 2\n\t"
      "v_cvt_pk_bf16_f32 %[t], %[zy], %[yp3]\n\t"
      "v_dot2_f32_bf16 %[zy], %[t], %[one], 0\n\t"
      "s_nop 2"
      : [t] "=&v"(t), [zy] "+v"(zy)
      : [yp0] "v"(yp[0]), [yp1] "v"(yp[1]), [yp2] "v"(yp[2]), [yp3] "v"(yp[3]), [one] "v"(kOnes));
}

__global__ __launch_bounds__(64) void wkv7_infer_bf16_kernel(InferBf16Params p) {
  __shared__ uint4 srow[kHead * 8];        // the state, 8 pieces of 16 bytes per row
  // the step's key-indexed operands: a, the rounded decay and r as product
  // words (key i's bf16 value in half i % 2), b and k as fp32
  __shared__ uint4 opw[3][kHead / 4];
  __shared__ float4 opf[2][kHead / 4];
  enum { O_A = 0, O_W, O_R };
  enum { O_B = 0, O_K };

  const int h = blockIdx.x, bi = blockIdx.y;
  const int lane = threadIdx.x;
  const int T = p.T;
  const int64_t tstride = (int64_t)p.H * kHead;
  const int64_t tok0 = ((int64_t)bi * T * p.H + h) * kHead + lane;
  // operands of step t, loaded one step ahead; step 0's are requested first,
  // before the slot and the state, so that their latency and the state's
  // overlap
  bool nlive = false;
  bf16_t nw = 0, na = 0, nb = 0, nk = 0, nr = 0, nv = 0;
  auto fetch = [&](int t) {
    nlive = !p.mask || (p.mask[(int64_t)bi * T + t] & 0x7fffu) != 0u;
    if (nlive) {
      const int64_t off = tok0 + (int64_t)t * tstride;
      nw = p.w[off]; na = p.a[off]; nb = p.b[off]; nk = p.k[off]; nr = p.r[off]; nv = p.v[off];
    }
  };
  if (T > 0) fetch(0);
  const int64_t slot = p.batch_ids[bi];
  // an out-of-range slot is refused: zero output, no state touched
  if (slot < 0 || slot >= p.full_batch) {
    for (int t = 0; t < T; ++t) p.y[tok0 + (int64_t)t * tstride] = 0;
    return;
  }
  const uint32_t elapsed = p.elapsed_t ? (uint32_t)p.elapsed_t[slot] : 0u;
  uint4* st = reinterpret_cast<uint4*>(p.state + (slot * p.H + h) * (kHead * kHead));
  // the state is read and written once, with the non-temporal hint as in the
  // fp32 kernel (measured at config[3] with the state read from HBM: 44.2 ->
  // 40.0 us; unchanged with one state buffer reused from the caches)
  typedef unsigned ntu4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const int u = m * 64 + lane;
    const ntu4 x = __builtin_nontemporal_load(reinterpret_cast<const ntu4*>(st) + u);
    srow[rot_piece(u >> 3, u & 7)] = make_uint4(x.x, x.y, x.z, x.w);
  }
  __syncthreads();
  // the row as it is stored: keys 2 m and 2 m + 1 in the low and high half of
  // sp[m]
  uint32_t sp[kHead / 2];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const uint4 x = srow[rot_piece(lane, q)];
    sp[4 * q + 0] = x.x;
    sp[4 * q + 1] = x.y;
    sp[4 * q + 2] = x.z;
    sp[4 * q + 3] = x.w;
  }

  uint32_t valid_t = 0;
  uint32_t* const opwu = reinterpret_cast<uint32_t*>(opw);
  float* const opff = reinterpret_cast<float*>(opf);
  const int half = 16 * (lane & 1);        // this lane's key in its word
  for (int t = 0; t < T; ++t) {
    const int64_t off = tok0 + (int64_t)t * tstride;
    const bool live = nlive;
    const bf16_t cw = nw, ca = na, cb = nb, ck = nk, cr = nr, cv = nv;
    if (t + 1 < T) fetch(t + 1);
    if (!live) {   // uniform: the mask entry is one per (row, step)
      p.y[off] = 0;
      continue;
    }
    float wd = decay_f(sigmoid_f(bf16_to_f32(cw)));
    if (p.use_dither) wd += dither_f(elapsed + valid_t);
    __syncthreads();   // the previous step's reads of the operands are done
    opwu[O_A * kHead + lane] = (uint32_t)ca << half;
    opwu[O_W * kHead + lane] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)wd) << half;
    opwu[O_R * kHead + lane] = (uint32_t)cr << half;
    opff[O_B * kHead + lane] = bf16_to_f32(cb);
    opff[O_K * kHead + lane] = bf16_to_f32(ck);
    const float vj = bf16_to_f32(cv);
    __syncthreads();
    // Running sums are kept unrounded (z): the reference's bf16 sum after key
    // i is rb(z_i), and z_{i+1} = rb(z_i) + rb(product_{i+1}) in fp32, so
    // sa_{i+1} = rb(sa_i + rb(a_{i+1} S[j, i+1])) as kernel.rs:81-83 has it.
    float z = 0.0f;
    float pz[4];
    sa_products(sp[0], sp[1], opw[O_A][0], pz);
#pragma unroll
    for (int i4 = 0; i4 < kHead / 4; ++i4) {
      float pn[4];
      if (i4 + 1 < kHead / 4) {
        sa_four<true>(pz, sp[2 * i4 + 2], sp[2 * i4 + 3], opw[O_A][i4 + 1], pn, z);
#pragma unroll
        for (int e = 0; e < 4; ++e) pz[e] = pn[e];
      } else {
        sa_four<false>(pz, 0u, 0u, uint4{}, pn, z);
      }
    }
    const float sa = rb(z);
    float zy = 0.0f;
    float yq[4] = {0.f, 0.f, 0.f, 0.f};   // the previous four keys' products with r
#pragma unroll
    for (int i4 = 0; i4 < kHead / 4; ++i4) {
      const uint4 w4 = opw[O_W][i4], r4 = opw[O_R][i4];
      const float4 b4 = opf[O_B][i4], k4 = opf[O_K][i4];
      // S[j,i] = rb(rb(rb(S w) + rb(sa b)) + rb(k v)) for keys 4 i4 .. + 3
      const float sb[4] = {sa * b4.x, sa * b4.y, sa * b4.z, sa * b4.w};
      const float kvv[4] = {k4.x * vj, k4.y * vj, k4.z * vj, k4.w * vj};
      float yn[4];
      if (i4 == 0)
        update_four<false>(sp[0], sp[1], w4, sb, kvv, r4, yq, yn, zy);
      else
        update_four<true>(sp[2 * i4], sp[2 * i4 + 1], w4, sb, kvv, r4, yq, yn, zy);
#pragma unroll
      for (int e = 0; e < 4; ++e) yq[e] = yn[e];
    }
    y_links(yq, zy);
    const float y = rb(zy);
    p.y[off] = (bf16_t)(__float_as_uint(y) >> 16);
    ++valid_t;
  }

  // write the rows back through LDS: coalesced 16-byte stores
  __syncthreads();
#pragma unroll
  for (int q = 0; q < 8; ++q) srow[rot_piece(lane, q)] = make_uint4(sp[4 * q], sp[4 * q + 1], sp[4 * q + 2], sp[4 * q + 3]);
  __syncthreads();
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const int u = m * 64 + lane;
    const uint4 x = srow[rot_piece(u >> 3, u & 7)];
    __builtin_nontemporal_store(ntu4{x.x, x.y, x.z, x.w}, reinterpret_cast<ntu4*>(st) + u);
  }
}

hipError_t launch_infer_bf16(const InferDesc& d, hipStream_t stream) {
  InferBf16Params p;
  p.w = static_cast<const bf16_t*>(d.w);
  p.r = static_cast<const bf16_t*>(d.r);
  p.k = static_cast<const bf16_t*>(d.k);
  p.v = static_cast<const bf16_t*>(d.v);
  p.a = static_cast<const bf16_t*>(d.a);
  p.b = static_cast<const bf16_t*>(d.b);
  p.batch_ids = d.batch_ids;
  p.state = static_cast<bf16_t*>(d.state);
  p.mask = static_cast<const bf16_t*>(d.context_mask);
  p.elapsed_t = d.elapsed_t;
  p.y = static_cast<bf16_t*>(d.y);
  p.T = d.T;
  p.H = d.H;
  p.full_batch = d.full_batch;
  p.use_dither = d.use_dither;
  hipLaunchKernelGGL(wkv7_infer_bf16_kernel, dim3(d.H, d.Ba, 1), dim3(64, 1, 1), 0, stream, p);
  return hipGetLastError();
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
  p.state = static_cast<float*>(d.state);
  p.mask = static_cast<const Tin*>(d.context_mask);
  p.y = static_cast<Tin*>(d.y);
  p.T = d.T;
  p.H = d.H;
  p.full_batch = d.full_batch;
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
  if (d.state_dtype == Dtype::BF16) return launch_infer_bf16(d, stream);
  return d.dtype == Dtype::BF16 ? launch_infer_t<bf16_t>(d, stream) : launch_infer_t<float>(d, stream);
}

}  // namespace wkv7
