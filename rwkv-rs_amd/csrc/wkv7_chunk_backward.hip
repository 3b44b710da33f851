// Chunked WKV7 backward on the matrix cores (bf16 operands, fp32 state and
// gradients of the state).
//
// Computes what wkv7_backward_kernel does (crates/rwkv-nn/src/kernels/
// wkv7_common/kernel.rs:116-308, launched by wkv7_common/host.rs:185-369):
// the six input gradients and the initial-state gradient from the forward's
// 16-step checkpoints and removal_state. It works on the matrix form of each
// 16-step chunk (wkv7_chunk.hpp). With the chunk's start state S0 (the
// previous checkpoint) and the gradient dS arriving from the later chunks,
// and writing dS' = dS diag(gamma_L):
//   dSA   = P^T (B~ dS'^T + A_rb^T dY)                 (dsa_t = dS_t b_t)
//   dS0^T = dS'^T + R^^T dY + A^^T dSA                  (carried to chunk c-1)
//   dV    = K~ dS'^T + A_rk^T dY + A_ak^T dSA
//   dK    = (V dS' + B_yv R^ + B_sav A^) / gamma_t
//   dB    = (SA dS' + B_ysa R^ + B_sasa A^) / gamma_t
//   dR    = gamma_t (dY S0 + C_dyv K~ + C_dysa B~)
//   dA    = gamma_{t-1} (dSA S0 + C_dsav K~ + C_dsasa B~)
// with the step-by-step products B_yv[t][s] = v_t.dy_s (s >= t),
// B_sav = v_t.dsa_s (s > t), B_ysa = sa_t.dy_s (s >= t), B_sasa = sa_t.dsa_s
// (s > t) and C_xy[t][s] = x_t.y_s for s <= t (s < t for dsa). The decay
// gradient follows from the log-decay prefix g_t: dL/dg_t = r_t dr_t -
// k_t dk_t - b_t db_t + a_{t+1} da_{t+1} (+ E at the chunk's last step, E =
// sum_s (K~ o V dS')_s + (B~ o SA dS')_s + sum_j S0 o dS'), and
// dw_u = W_SCALE sigmoid(x_u)(1 - sigmoid(x_u)) sum_{t>=u} dL/dg_t.
// Chunk 0's start state is rebuilt the way the reference rebuilds every step
// (divide by the decay, kernel.rs:239-246); the other chunks read it from the
// previous checkpoint. With chunk_len > 16 only every (chunk_len / 16)-th
// chunk starts at a checkpoint; the set-up waves rebuild the others' start
// states by the same reversal, from the end state the next chunk started
// with, carried in registers.
//
// Work layout: one workgroup of eight waves per (batch, head), two per SIMD,
// chunks in reverse order. Waves 0-3 ("gradient waves", wave w owns value
// tile w and key tile w) carry the state gradient; waves 4-7 ("set-up
// waves", key tile w - 4) do the per-chunk work that does not depend on it,
// one chunk ahead, so each SIMD interleaves two instruction streams:
//   phase A: gradient waves: state-gradient chain and dV of chunk c; set-up
//            waves: staging loads, the finished decay gradient of chunk c+1,
//            the step products of v, dy, sa of chunk c (one per wave), and
//            the decays and decayed rows of chunk c-1 (keys of their own
//            slice and of their SIMD's gradient wave)
//   phase B: gradient waves: gradient flush of chunk c+1, the step products
//            with dSA of chunk c; set-up waves: step products of the decayed
//            rows of chunk c-1 and P = (I - A_ab)^-1 (wave 4), staging stores
//   phase C: key-indexed gradients of chunk c, key tile w: dK, dB and their
//            part of the decay gradient on the gradient wave, dR, dA and the
//            rest on the set-up wave, which finishes dw after the barrier
// Phase C's operands that phase B does not write are read at the end of
// phase B, so their latency overlaps the barrier; sums over the four quads of
// a wave use gfx950's row-swapping moves instead of LDS.
// Within a phase each wave first issues its LDS reads, then computes. Inputs
// are staged through registers, loaded in phase A and written to LDS in
// phase B: the rows only the decays read (x, r, k, a, b) in one buffer, two
// chunks ahead; v, dy and the removal_state (split into bf16 hi/lo rows once,
// when staged) in two, one chunk ahead.
#include <type_traits>

#include "wkv7_chunk.hpp"
#include "wkv7_launch.hpp"

namespace wkv7 {
namespace {

using namespace chunk;

constexpr int kWaves = 8;
constexpr int kBlock = 64 * kWaves;
constexpr int kGradWaves = 4;          // waves 0-3: gradients; 4-7: set-up of the next chunk
constexpr int kSetup = 64 * 4;         // threads of either group of four waves
enum { I_X, I_R, I_K, I_A, I_B, I_V, I_DY, I_COUNT };   // input tensors
constexpr int kDecayIn = 5;                             // I_X..I_B: read by the decays only
enum { S_V, S_DY, S_SAH, S_SAL, S_COUNT };              // rows read by the gradients
enum { T_AH, T_AL, T_RH, T_RL, T_KH, T_KL, T_BH, T_BL, T_COUNT };   // decayed rows, hi/lo
enum { F_AKT, F_RBT, F_RKT, F_PT, F_COUNT };            // stacked operands from the decayed rows
enum { G_BYV, G_CDYV, G_BYSA, G_CDYSA, G_BSAV, G_CDSAV, G_BSASA, G_CDSASA, G_COUNT };
enum { O_DV, O_DK, O_DB, O_DR, O_DA, O_DW, O_COUNT };   // staged gradient tiles
constexpr int kOutRounds = O_COUNT * kL * 8 / kSetup;          // 16-byte stores per set-up thread
constexpr int kDecayPieces = kDecayIn * kL * 8;                // 16-byte pieces per chunk
constexpr int kDecayRounds = (kDecayPieces + kSetup - 1) / kSetup;
constexpr float kSigFromLw2 = 1.0f / (kWScale * kLog2e);        // sigmoid = lw2 * this
static_assert(2 * kL * 8 == kSetup, "v and dy rows: one 16-byte piece per set-up thread");
static_assert(kL * 16 == kSetup, "removal_state rows: four values per set-up thread");
static_assert(O_COUNT * kL * 8 % kSetup == 0, "whole rounds of gradient stores");

// per-chunk set-up, double-buffered (chunk c & 1)
struct Prep {
  PadTile rows[T_COUNT];            // decayed rows, rotated
  float gT[64][kL + 4];             // log2 prefix decay, [key][step]
  float lwT[64][kL + 4];            // log2 step decay, [key][step]
  float gl[64];                     // gamma_L
  bf16x8 frag[F_COUNT][64];         // stacked 16x16 operands
};

struct BwdLds {
  PadTile dec[kDecayIn];            // x, r, k, a, b rows of the next chunk to set up
  PadTile stg[2][S_COUNT];          // v, dy, sa hi, sa lo rows, double-buffered
  Prep prep[2];                     // chunk 0 also keeps its rebuilt start state in prep[1]
  bf16x8 frag[G_COUNT][64];         // step products with v, dy, sa, dsa (stacked)
  bf16_t xds[2][64][64];            // dS' hi/lo, [value j][key i]
  bf16_t xdsa[2][64][kL];           // dSA hi/lo, [value j][step t]
  f32x4 kx[4][64];                  // the gradient waves' part of the decay gradient, per key tile
  bf16_t outs[2][O_COUNT][kL][64];  // a chunk's bf16 gradients, written out as whole rows (out_at), double-buffered
  bf16_t zero[kL][64];              // an all-zero row tile
  // chunk_len > 16: the chunk whose start state is rebuilt next (staged with
  // its gradient rows): the removal_state in fp32, and the k and b rows
  float sa32[kL][64];
  PadTile kbt[2];
  float abt[kL][20];                // A_ab on its way to A_ab^T (set-up wave 4; rows padded so
                                    // the four quads' column writes fall on distinct banks)
};
typedef float S0Rows[64][68];       // chunk 0's rebuilt start state, [key i][value j]
static_assert(sizeof(S0Rows) <= sizeof(Prep), "start state fits the free set-up buffer");

struct BwdChunkParams {
  const bf16_t* in[I_COUNT];   // [B,T,H,64] each
  const float* ckpt;           // [B,H,T/16,64(key),64(value)]
  const float* sa;             // [B,T,H,64]
  const float* dsT;            // [B,H,64(value),64(key)] or null
  bf16_t* dw;                  // gradients [B,T,H,64]
  bf16_t* dr;
  bf16_t* dk;
  bf16_t* dv;
  bf16_t* da;
  bf16_t* db;
  float* ds0;                  // [B,H,64,64] or null
  int T, H;
  int C;                       // chunk_len: a multiple of 16
};

// element (row, key) of a staged gradient tile: 16-byte pieces rotated by
// two per group of four rows, so the four quads of a wave, which write rows
// 4 qd + r, hit disjoint banks
__device__ __forceinline__ bf16_t& out_at(bf16_t (*tile)[64], int row, int key) {
  return tile[row][8 * (((key >> 3) + 2 * ((row >> 2) & 3)) & 7) + (key & 7)];
}
// 4-value piece q (steps 4 q .. 4 q + 3) of row j of a dSA exchange tile
// ([value j][step], 32-byte rows): pieces rotated by (j / 8) % 4, so the
// writes of 16 consecutive rows spread over the banks (unrotated: four-way
// conflicts), while the transposed reads still take 4 whole rows per 16 lanes
__device__ __forceinline__ bf16_t* xdsa_at(bf16_t (*tile)[kL], int j, int q) {
  return &tile[j][4 * ((q + (j >> 3)) & 3)];
}
__device__ __forceinline__ f32x4 widen4(bf16x4 x) { return __builtin_convertvector(x, f32x4); }
__device__ __forceinline__ bf16x8 stack_f(f32x4 x) { return stack(split4(x)); }
// 16x16 product of two row fragment pairs over the 64 columns (k = column)
__device__ __forceinline__ f32x4 gram_x3(const Split8 (&a)[2], const Split8 (&b)[2]) {
  f32x4 c = {0.f, 0.f, 0.f, 0.f};
  c = mma32x3(a[0], b[0], c);
  return mma32x3(a[1], b[1], c);
}
__device__ __forceinline__ Split8 row_pair(const bf16_t (*hi)[64], const bf16_t (*lo)[64], int t, int m, int qd) {
  return Split8{row_frag(hi, t, m, qd), row_frag(lo, t, m, qd)};
}
__device__ __forceinline__ float hi_lo(bf16x4 h, bf16x4 l, int r) { return (float)h[r] + (float)l[r]; }

// The checkpoints and removal_state are read once and the gradients written
// once per launch: those accesses carry the non-temporal hint (measured: about
// 1.5% faster at config[1]; the same hint on the forward's checkpoint stores
// made the forward 18% slower, so the forward does not use it).
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// ---- set-up of one chunk, step 1: decays and decayed rows. Each of the 8
// waves takes keys 8 w .. 8 w + 7, two per lane (keys 8 w + 2 qd, + 1).
struct DecayIn { uint32_t x, a, r, k, b; };   // two bf16 each
__device__ __forceinline__ uint32_t read2(const bf16_t (*tile)[64], int row, int c) {
  return *reinterpret_cast<const uint32_t*>(tile_at(tile, row, c));
}
__device__ __forceinline__ void write2(bf16_t (*tile)[64], int row, int c, uint32_t v) {
  *reinterpret_cast<uint32_t*>(tile_at(tile, row, c)) = v;
}
__device__ __forceinline__ DecayIn decay_load(const PadTile* dec, int wave, int t, int qd) {
  const int c0 = 8 * wave + 2 * qd;
  return DecayIn{read2(dec[I_X].r, t, c0), read2(dec[I_A].r, t, c0), read2(dec[I_R].r, t, c0),
                 read2(dec[I_K].r, t, c0), read2(dec[I_B].r, t, c0)};
}
__device__ __forceinline__ float bf_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
__device__ __forceinline__ void setup_decays(Prep& P, const DecayIn& in, int wave, int t, int qd) {
  const int c0 = 8 * wave + 2 * qd;
  // plain float arrays around the cross-lane (DPP) operations: this compiler
  // folds DPP builtins whose source is an element of an ext_vector value into
  // a single one (all elements get element 0's)
  const float xs[2] = {bf_lo(in.x), bf_hi(in.x)};
  float g2[2], lw2[2], gam[2], gin[2], gpv[2], gL[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    lw2[e] = log2_decay(xs[e]);
    g2[e] = row_scan16(lw2[e]);
    gam[e] = exp2_f(g2[e]);
    gin[e] = exp2_f(-g2[e]);
    gpv[e] = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
        __builtin_bit_cast(int, 1.0f), __builtin_bit_cast(int, gam[e]), 0x111, 0xf, 0xf, false));
    gL[e] = row_last16(gam[e]);
  }
  uint32_t hi, lo;
  split2(bf_lo(in.a) * gpv[0], bf_hi(in.a) * gpv[1], hi, lo);
  write2(P.rows[T_AH].r, t, c0, hi);
  write2(P.rows[T_AL].r, t, c0, lo);
  split2(bf_lo(in.r) * gam[0], bf_hi(in.r) * gam[1], hi, lo);
  write2(P.rows[T_RH].r, t, c0, hi);
  write2(P.rows[T_RL].r, t, c0, lo);
  split2(bf_lo(in.k) * gin[0], bf_hi(in.k) * gin[1], hi, lo);
  write2(P.rows[T_KH].r, t, c0, hi);
  write2(P.rows[T_KL].r, t, c0, lo);
  split2(bf_lo(in.b) * gin[0], bf_hi(in.b) * gin[1], hi, lo);
  write2(P.rows[T_BH].r, t, c0, hi);
  write2(P.rows[T_BL].r, t, c0, lo);
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    P.gT[c0 + e][t] = g2[e];
    P.lwT[c0 + e][t] = lw2[e];
  }
  if (t == 0) {
    P.gl[c0] = gL[0];
    P.gl[c0 + 1] = gL[1];
  }
}

// ---- set-up step 2: one step-by-step product of decayed rows per wave.
// wave 0: A_ab and A_ab^T, and from them P = (I - A_ab)^-1 on the matrix
// cores (registers only, no LDS round trips); 1: A_ak^T; 2: A_rb^T; 3: A_rk^T.
struct GramIn { Split8 X[2], Y[2]; };
__device__ __forceinline__ GramIn products_load(const Prep& P, int wave, int t, int qd) {
  const int xa = wave < 2 ? T_AH : T_RH;
  const int yb = (wave & 1) ? T_KH : T_BH;
  GramIn g;
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    g.X[m] = row_pair(P.rows[xa].r, P.rows[xa + 1].r, t, m, qd);
    g.Y[m] = row_pair(P.rows[yb].r, P.rows[yb + 1].r, t, m, qd);
  }
  return g;
}
__device__ __forceinline__ void setup_products(Prep& P, const GramIn& g, int wave, int t, int qd, int lane,
                                               float (*abt)[20]) {
  const int strict = wave < 2 ? 1 : 0;
  const Split8 (&X)[2] = g.X;
  const Split8 (&Y)[2] = g.Y;
  f32x4 d = gram_x3(X, Y);   // [t'][s] = x_t' . y_s, lane column s = t
#pragma unroll
  for (int r = 0; r < 4; ++r) d[r] = 4 * qd + r - t >= strict ? d[r] : 0.f;
  if (wave == 0) {
    // d = A_ab[t'][s]; A_ab^T in the same layout through LDS (this wave
    // writes its result tile and reads it back by rows)
#pragma unroll
    for (int r = 0; r < 4; ++r) abt[4 * qd + r][t] = d[r];
    wave_lds_sync();
    const f32x4 dt = *reinterpret_cast<const f32x4*>(&abt[t][4 * qd]);
    // P^T as an A operand: lane l holds P[4 qd + e][l % 16], P's result layout
    P.frag[F_PT][lane] = stack_f(unit_lower_inverse(d, dt, t, qd));
  } else {
    P.frag[wave - 1][lane] = stack_f(d);
  }
}

// kLong: chunk_len > 16. Only every (chunk_len / 16)-th start state is a
// checkpoint; the others are rebuilt by the reference's reversal (see
// reverse_chunk), on the set-up waves.
template <bool kLong>
__global__ __launch_bounds__(kBlock, 1) void wkv7_bwd_chunk_kernel(const BwdChunkParams p) {
  __shared__ BwdLds L;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
  const bool grad = wave < kGradWaves;   // gradient waves 0-3, set-up waves 4-7
  const int wq = wave & 3;               // value tile / key tile / key slice of the wave
  const int utid = tid & (kSetup - 1);   // thread index within its group of four waves
  const int t = lane & 15, qd = lane >> 4;
  const int h = blockIdx.x, b = blockIdx.y, H = p.H, T = p.T;
  const int64_t bh = (int64_t)b * H + h;
  const int64_t tstride = (int64_t)H * kHead;
  const int64_t tok0 = ((int64_t)b * T * H + h) * kHead;
  const int nchunks = T / kL;
  const int q = kLong ? p.C / kL : 1;   // 16-step chunks per checkpoint
  const float* const ckbh = p.ckpt + bh * (T / (kL * q)) * (kHead * kHead);

  // ---- staging through registers (set-up waves). bf16 rows as rotated
  // pieces: piece p = 256 k + utid is row (p / 8) % 16, slot p % 8 of input
  // p / 128, whose index is wave-uniform, so its pointer stays in scalar
  // registers. The removal_state: thread utid holds row utid / 16, values
  // 4 (utid % 16) .. + 3.
  struct Pre { uint4 dec[kDecayRounds]; uint4 vy; f32x4 sa; uint4 kb; };
  // the sources, chosen once (waves 6 and 7 have no piece in the last decay
  // round: they load input 4's again and do not stage it)
  const bf16_t* src[kDecayRounds + 1];
#pragma unroll
  for (int k = 0; k < kDecayRounds; ++k) {
    const int in = 2 * k + (wq >> 1);
    src[k] = p.in[in < kDecayIn ? in : kDecayIn - 1] + tok0;
  }
  src[kDecayRounds] = p.in[I_V + (wq >> 1)] + tok0;
  const bf16_t* const kb_src = p.in[(wq >> 1) ? I_B : I_K] + tok0;   // k rows, then b rows
  const float* const sa_src = p.sa + tok0 + (int64_t)(utid >> 4) * tstride + 4 * (utid & 15);
  // piece offset within a chunk: row (utid / 8) % 16, rotated slot
  const int64_t piece_off = (int64_t)((utid >> 3) & 15) * tstride + 8 * (((utid & 7) - tile_rot((utid >> 3) & 15)) & 7);
  auto fetch = [&](int cdec, int cg) {   // chunk of the decay rows, chunk of the gradient rows
    Pre pr;
    const int64_t od = (int64_t)kL * cdec * tstride + piece_off;
#pragma unroll
    for (int k = 0; k < kDecayRounds; ++k) pr.dec[k] = *reinterpret_cast<const uint4*>(src[k] + od);
    pr.vy = *reinterpret_cast<const uint4*>(src[kDecayRounds] + (int64_t)kL * cg * tstride + piece_off);
    pr.sa = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(sa_src + (int64_t)kL * cg * tstride));
    if constexpr (kLong) pr.kb = *reinterpret_cast<const uint4*>(kb_src + (int64_t)kL * cg * tstride + piece_off);
    return pr;
  };
  auto stage_dec = [&](const Pre& pr) {
#pragma unroll
    for (int k = 0; k < kDecayRounds; ++k)
      if (2 * k + (wq >> 1) < kDecayIn) {
        const int piece = kSetup * k + utid;   // 128 pieces per input
        reinterpret_cast<uint4*>(&L.dec[piece >> 7].r[0][0])[piece & 127] = pr.dec[k];
      }
  };
  auto stage_grad = [&](const Pre& pr, int sb) {
    reinterpret_cast<uint4*>(&L.stg[sb][utid >> 7].r[0][0])[utid & 127] = pr.vy;   // v rows, then dy rows
    const Split4 s = split4(pr.sa);
    write4(L.stg[sb][S_SAH].r, utid >> 4, 4 * (utid & 15), s.hi);
    write4(L.stg[sb][S_SAL].r, utid >> 4, 4 * (utid & 15), s.lo);
    if constexpr (kLong) {
      // single-buffered: read in phase A of the chunk, written in phase B of
      // the one after it
      reinterpret_cast<uint4*>(&L.kbt[utid >> 7].r[0][0])[utid & 127] = pr.kb;
      *reinterpret_cast<f32x4*>(&L.sa32[utid >> 4][4 * (utid & 15)]) = pr.sa;
    }
  };

  // ---- state gradient (gradient waves): value tile jb = wq, key tiles ib,
  // result layout (rows = key i = 16 ib + 4 qd + r, columns = value j = 16 jb + t)
  const int jb = wq, jcol = 16 * jb + t;
  f32x4 dS[4];
#pragma unroll
  for (int ib = 0; ib < 4; ++ib) {
    if (grad && p.dsT)
      dS[ib] = *reinterpret_cast<const f32x4*>(p.dsT + bh * (kHead * kHead) + jcol * kHead + 16 * ib + 4 * qd);
    else
      dS[ib] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const int ki = 16 * wq + t;   // key of the lane in the key-gradient stage (column of its tile)

  // start state S0 of chunk c >= 1 (the checkpoint of chunk c - 1) as the
  // rows [key ki][value 32 m + 4 qd .., + 16 ..] of the key stage; loaded at
  // the start of the chunk, used two phases later
  auto load_ckpt = [&](int n, f32x4 (&rowv)[2][2]) {   // checkpoint n
    const float* ck = ckbh + (int64_t)n * (kHead * kHead);
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      rowv[m][0] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(ck + ki * kHead + 32 * m + 4 * qd));
      rowv[m][1] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(ck + ki * kHead + 32 * m + 16 + 4 * qd));
    }
  };
  // start state of chunk c, c a multiple of q
  auto load_s0 = [&](int c, f32x4 (&rowv)[2][2]) { load_ckpt(c / q - 1, rowv); };
  // kLong: the start state of chunk c from its end state Se by the
  // reference's reversal over the chunk's 16 steps (kernel.rs:239-246),
  // S_{t-1} = (S_t - k_t v_t^T - b_t sa_t^T) / w~_t, in the key stage's
  // layout (the lane's key ki, values 32 m + 16 h + 4 qd + e): one decay per
  // lane and step. Every operand from LDS: v from the staged gradient rows,
  // k, b and the fp32 removal_state from their own staging, log2 w~ from the
  // set-up of chunk c.
  auto reverse_chunk = [&](int c, const Prep& P, const PadTile* stg, const f32x4 (&Se)[2][2],
                           f32x4 (&S)[2][2]) {
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      S[m][0] = Se[m][0];
      S[m][1] = Se[m][1];
    }
#pragma unroll 4
    for (int tt = kL - 1; tt >= 0; --tt) {
      const float kv = __uint_as_float((uint32_t)*tile_at(L.kbt[0].r, tt, ki) << 16);
      const float bv = __uint_as_float((uint32_t)*tile_at(L.kbt[1].r, tt, ki) << 16);
      const float winv = exp2_f(-P.lwT[ki][tt]);
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int j0 = 32 * m + 16 * hh + 4 * qd;
          const f32x4 vv = widen4(read4(stg[S_V].r, tt, j0));
          const f32x4 sv = *reinterpret_cast<const f32x4*>(&L.sa32[tt][j0]);
#pragma unroll
          for (int e = 0; e < 4; ++e) S[m][hh][e] = (S[m][hh][e] - kv * vv[e] - bv * sv[e]) * winv;
        }
    }
  };
  // kLong, set-up waves: the start state of the chunk processed last, i.e.
  // the end state of the next one (the last checkpoint before the loop)
  f32x4 Snext[2][2];
  if (kLong && !grad) load_ckpt(T / (kL * q) - 1, Snext);

  // the staged gradient tiles of chunk cc to memory (gradient waves in the
  // loop, whose phase B is the shorter one; set-up waves after it): thread
  // utid writes 16-byte pieces p = 256 k + utid (tile p / 128, row (p / 8) %
  // 16); tile 2 k + wq / 2 is wave-uniform, so the destination is picked by
  // scalar selects and stays a global pointer
  bf16_t* dst[kOutRounds];
#pragma unroll
  for (int k = 0; k < kOutRounds; ++k) {
    const int tile = 2 * k + (wq >> 1);
    bf16_t* const q = tile == O_DV ? p.dv : tile == O_DK ? p.dk : tile == O_DB ? p.db
                    : tile == O_DR ? p.dr : tile == O_DA ? p.da : p.dw;
    dst[k] = q + tok0 + (int64_t)((utid >> 3) & 15) * tstride + 8 * (utid & 7);
  }
  auto flush = [&](int cc) {
#pragma unroll
    for (int k = 0; k < kOutRounds; ++k) {
      const int tile = 2 * k + (wq >> 1), row = (utid >> 3) & 15;
      const uint4 v = *reinterpret_cast<const uint4*>(&out_at(L.outs[cc & 1][tile], row, 8 * (utid & 7)));
      __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4*>(dst[k] + (int64_t)kL * cc * tstride));
    }
  };

  // the decay gradient of chunk cc, finished by the set-up wave of key tile
  // wq from its own part (carried in registers) and the gradient wave's part
  f32x4 carry = {0.f, 0.f, 0.f, 0.f}, sig = carry;
  auto finish = [&](int cc) {
    const f32x4 kpart = L.kx[wq][lane];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float dwv = (carry[r] - kpart[r]) * kWScale * sig[r] * (1.0f - sig[r]);
      out_at(L.outs[cc & 1][O_DW], 4 * qd + r, ki) = __builtin_bit_cast(bf16_t, (__bf16)dwv);
    }
  };

  // Issue priority: when both waves of a SIMD can issue, the set-up wave goes
  // first. Its phases are the longer ones (phase C's decay-gradient terms,
  // phase B's products), so the gradient wave fills the gaps instead of the
  // set-up wave waiting behind it (measured: 1.04 -> 0.98-0.99 ms at
  // config[1]; the level and per-phase switching made no further difference).
  if (!grad) __builtin_amdgcn_s_setprio(2);

  // ---- prologue: set up the last chunk (set-up waves)
  const int last = nchunks - 1;
  if (!grad) {
    reinterpret_cast<uint2*>(&L.zero[0][0])[utid] = make_uint2(0, 0);
    const Pre pr = fetch(last, last);
    stage_dec(pr);
    stage_grad(pr, last & 1);
  }
  lds_barrier();
  setup_decays(L.prep[last & 1], decay_load(L.dec, wave, t, qd), wave, t, qd);
  lds_barrier();
  if (!grad) {
    if (last >= 1) stage_dec(fetch(last - 1, last));
    setup_products(L.prep[last & 1], products_load(L.prep[last & 1], wq, t, qd), wq, t, qd, lane, L.abt);
  }

  // one chunk; kFull: chunk c - 1 exists and is set up alongside (c >= 1).
  // The last iteration (c == 0) is peeled.
  auto run_chunk = [&](const int c, auto full) {
    constexpr bool kFull = decltype(full)::value;
    const int sb = c & 1;
    Prep& P = L.prep[sb];
    Prep& Pn = L.prep[sb ^ 1];   // set-up of chunk c - 1
    const PadTile* const stg = L.stg[sb];
    bf16_t (*const outs)[kL][64] = L.outs[sb];
    S0Rows& s0r = *reinterpret_cast<S0Rows*>(&L.prep[1]);   // used at c == 0 only
    lds_barrier();

    // ================= phase A
    Pre pre;
    f32x4 S0row[2][2];
    f32x4 dv;
    if (grad) {
      if constexpr (!kFull && !kLong) {
        // rebuild S0 by reversing the chunk's 16 steps from its checkpoint
        // (kernel.rs:239-246): S_{t-1} = (S_t - v_t k_t^T - sa_t b_t^T) / w~_t.
        // The decay-rows buffer still holds chunk 0's rows; sa in fp32 from memory.
        const float* ck = ckbh;
        f32x4 S0t[4];
#pragma unroll
        for (int ib = 0; ib < 4; ++ib)
#pragma unroll
          for (int r = 0; r < 4; ++r) S0t[ib][r] = ck[(16 * ib + 4 * qd + r) * kHead + jcol];
        for (int tt = kL - 1; tt >= 0; --tt) {
          const float vj = __uint_as_float((uint32_t)__builtin_bit_cast(uint16_t, *tile_at(stg[S_V].r, tt, jcol)) << 16);
          const float sj = p.sa[tok0 + (int64_t)tt * tstride + jcol];
#pragma unroll
          for (int ib = 0; ib < 4; ++ib) {
            const f32x4 kv = widen4(read4(L.dec[I_K].r, tt, 16 * ib + 4 * qd));
            const f32x4 bv = widen4(read4(L.dec[I_B].r, tt, 16 * ib + 4 * qd));
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float winv = exp2_f(-P.lwT[16 * ib + 4 * qd + r][tt]);
              S0t[ib][r] = (S0t[ib][r] - kv[r] * vj - bv[r] * sj) * winv;
            }
          }
        }
#pragma unroll
        for (int ib = 0; ib < 4; ++ib)
#pragma unroll
          for (int r = 0; r < 4; ++r) s0r[16 * ib + 4 * qd + r][jcol] = S0t[ib][r];
      }
      // the chain's LDS operands first, so their latency overlaps
      f32x4 glv[4];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) glv[ib] = *reinterpret_cast<const f32x4*>(&P.gl[16 * ib + 4 * qd]);
      const Split8 Bt0 = row_pair(P.rows[T_BH].r, P.rows[T_BL].r, t, 0, qd);
      const Split8 Bt1 = row_pair(P.rows[T_BH].r, P.rows[T_BL].r, t, 1, qd);
      const Split8 Kt0 = row_pair(P.rows[T_KH].r, P.rows[T_KL].r, t, 0, qd);
      const Split8 Kt1 = row_pair(P.rows[T_KH].r, P.rows[T_KL].r, t, 1, qd);
      const bf16x4 dycf = tr_frag(stg[S_DY].r, 0, 16 * jb, lane);   // dY[s][j] (k = s)
      const bf16x8 f_rbt = P.frag[F_RBT][lane], f_pt = P.frag[F_PT][lane];
      const bf16x8 f_rkt = P.frag[F_RKT][lane], f_akt = P.frag[F_AKT][lane];
      bf16x8 rT[4], aT[4];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
        rT[ib] = cat8(tr_frag(P.rows[T_RH].r, 0, 16 * ib, lane), tr_frag(P.rows[T_RL].r, 0, 16 * ib, lane));
        aT[ib] = cat8(tr_frag(P.rows[T_AH].r, 0, 16 * ib, lane), tr_frag(P.rows[T_AL].r, 0, 16 * ib, lane));
      }
      __builtin_amdgcn_sched_barrier(0);
      f32x4 dSp[4];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) dSp[ib] = dS[ib] * glv[ib];
      // the carried gradient's terms that do not wait for dSA first: dS'^T +
      // R^^T dY, so that dS' is not needed afterwards and is split in place
      f32x4 acc[4];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) acc[ib] = mma_s2(rT[ib], dycf, dSp[ib]);
      const Split8 Sx0 = split8(dSp[0], dSp[1]), Sx1 = split8(dSp[2], dSp[3]);
      f32x4 z = mma32x3(Bt0, Sx0, f32x4{0.f, 0.f, 0.f, 0.f});
      z = mma32x3(Bt1, Sx1, z);
      z = mma_s2(f_rbt, dycf, z);
      const f32x4 dsa = mma_s3(f_pt, split4(z), f32x4{0.f, 0.f, 0.f, 0.f});
      const Split4 dsas = split4(dsa);
      dv = mma32x3(Kt0, Sx0, f32x4{0.f, 0.f, 0.f, 0.f});
      dv = mma32x3(Kt1, Sx1, dv);
      dv = mma_s2(f_rkt, dycf, dv);
      dv = mma_s3(f_akt, dsas, dv);
      // carried gradient dS0^T = dS'^T + R^^T dY + A^^T dSA
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) dS[ib] = mma_s3(aT[ib], dsas, acc[ib]);
      // exchange for the key stage: dS' as [value j][key i], dSA as [j][step]
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const Split8& sx = m ? Sx1 : Sx0;
          write4(L.xds[0], jcol, 32 * m + 16 * hh + 4 * qd, half_of(sx.hi, hh));
          write4(L.xds[1], jcol, 32 * m + 16 * hh + 4 * qd, half_of(sx.lo, hh));
        }
      *reinterpret_cast<bf16x4*>(xdsa_at(L.xdsa[0], jcol, qd)) = dsas.hi;
      *reinterpret_cast<bf16x4*>(xdsa_at(L.xdsa[1], jcol, qd)) = dsas.lo;
    } else {
      if (c < last) finish(c + 1);
      if constexpr (kFull) {
        // at c == 1 the decay rows of chunk 0 are fetched again (harmless, and
        // the reversal of chunk 0 reads them)
        pre = fetch(c >= 2 ? c - 2 : 0, c - 1);
        if constexpr (!kLong) load_s0(c, S0row);
      }
      if constexpr (kLong) {
        if (kFull && c % q == 0) load_s0(c, S0row);
        else reverse_chunk(c, P, stg, Snext, S0row);
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          Snext[m][0] = S0row[m][0];
          Snext[m][1] = S0row[m][1];
        }
      }
      // step products of v, dy, sa of chunk c (one per wave), which do not
      // depend on the state gradient, as D = X1 Y1^T + X2 Y2^T:
      // B_yv^T = dy v^T (s >= t), C_dyv^T = v dy^T (s <= t),
      // B_ysa^T = dy sa^T (s >= t), C_dysa^T = sa dy^T (s <= t)
      {
        const int x1 = wq == 1 ? S_V : wq == 3 ? S_SAH : S_DY;
        const int y1 = wq == 0 ? S_V : wq == 2 ? S_SAH : S_DY;
        const int y2 = wq == 0 ? S_V : wq == 2 ? S_SAL : S_DY;
        const bf16_t (*const x2)[64] = wq == 2 ? stg[S_DY].r : wq == 3 ? stg[S_SAL].r : L.zero;
        bf16x8 px1[2], py1[2], px2[2], py2[2];
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          px1[m] = row_frag(stg[x1].r, t, m, qd);
          py1[m] = row_frag(stg[y1].r, t, m, qd);
          px2[m] = row_frag(x2, t, m, qd);
          py2[m] = row_frag(stg[y2].r, t, m, qd);
        }
        const int sgn = (wq & 1) ? -1 : 1;   // keep s >= t (B_), s <= t (C_)
        f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          d = mma32(px2[m], py2[m], d);
          d = mma32(px1[m], py1[m], d);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) d[r] = sgn * (4 * qd + r - t) >= 0 ? d[r] : 0.f;
        L.frag[G_BYV + wq][lane] = stack_f(d);
      }
      // decays and decayed rows of chunk c - 1, all 64 keys: the set-up
      // wave's own slice and that of the gradient wave of its SIMD
      if constexpr (kFull) {
        setup_decays(Pn, decay_load(L.dec, wave, t, qd), wave, t, qd);
        setup_decays(Pn, decay_load(L.dec, wq, t, qd), wq, t, qd);
      }
    }
    lds_barrier();

    // ================= phase B
    // dSA as row fragments (row = step t, k = value), from the [j][t] tiles
    auto dsa_frag = [&](int hl, int m) {
      return cat8(read_tr16(xdsa_at(L.xdsa[hl], 32 * m + 4 * qd + (t >> 2), t & 3)),
                  read_tr16(xdsa_at(L.xdsa[hl], 32 * m + 16 + 4 * qd + (t >> 2), t & 3)));
    };
    if (grad) {
      if (c < last) flush(c + 1);
#pragma unroll
      for (int r = 0; r < 4; ++r) out_at(outs[O_DV], 4 * qd + r, jcol) = __builtin_bit_cast(bf16_t, (__bf16)dv[r]);
      // step products with dSA: B_sav^T = dsa v^T (s > t), C_dsav^T = v dsa^T
      // (s < t), B_sasa^T = dsa sa^T (s > t), C_dsasa^T = sa dsa^T (s < t).
      // Wave 0 forms none: its SIMD also runs set-up wave 4, which forms the
      // inverse in this phase. Wave 1 forms both products with v (the two
      // orientations of the same operands), waves 2 and 3 one each with sa.
      if (wq != 0) {
        const Split8 q[2] = {{dsa_frag(0, 0), dsa_frag(1, 0)}, {dsa_frag(0, 1), dsa_frag(1, 1)}};
        Split8 g[2];
        {
          const bf16_t (*const ylo)[64] = wq >= 2 ? stg[S_SAL].r : L.zero;
          const int yhi = wq >= 2 ? S_SAH : S_V;
#pragma unroll
          for (int m = 0; m < 2; ++m) g[m] = Split8{row_frag(stg[yhi].r, t, m, qd), row_frag(ylo, t, m, qd)};
        }
        __builtin_amdgcn_sched_barrier(0);
        const int sgn = (wq & 1) ? -1 : 1;   // keep s > t (B_), s < t (C_)
        // the wave's orientation (wq is wave-uniform: a scalar branch)
        f32x4 e = {0.f, 0.f, 0.f, 0.f};
        if (wq & 1) {
          e = mma32x3(g[0], q[0], e);
          e = mma32x3(g[1], q[1], e);
        } else {
          e = mma32x3(q[0], g[0], e);
          e = mma32x3(q[1], g[1], e);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) e[r] = sgn * (4 * qd + r - t) > 0 ? e[r] : 0.f;
        L.frag[G_BSAV + wq][lane] = stack_f(e);
        if (wq == 1) {   // B_sav for wave 0
          f32x4 e0 = {0.f, 0.f, 0.f, 0.f};
          e0 = mma32x3(q[0], g[0], e0);
          e0 = mma32x3(q[1], g[1], e0);
#pragma unroll
          for (int r = 0; r < 4; ++r) e0[r] = (4 * qd + r - t) > 0 ? e0[r] : 0.f;
          L.frag[G_BSAV][lane] = stack_f(e0);
        }
      }
    } else {
      if constexpr (kFull) {
        // the decayed rows first: the staging waits for phase A's global loads
        const GramIn gi = products_load(Pn, wq, t, qd);
        __builtin_amdgcn_sched_barrier(0);
        stage_dec(pre);             // decay rows of chunk c - 2 (the decays of phase A are done)
        stage_grad(pre, sb ^ 1);    // gradient rows of chunk c - 1 (free buffer)
        setup_products(Pn, gi, wq, t, qd, lane, L.abt);
      }
    }
    // Phase C's operands that phase B does not write, read before the
    // barrier so that their latency overlaps the wait (the decayed rows and
    // the step products with v, dy, sa of chunk c, dS' and dSA from phase A,
    // the staged rows); only the products with dSA from phase B are read after.
    const int kb = wq;
    Split4 Rc, Ac, Kc, Bc;   // decayed rows as B operands (k = step, column = key), split
    Split8 Db[2];            // dS' as B operand (k = value j, column = key ki)
    f32x4 g4;
    bf16x8 cv0, cv1, f_b0, f_b1;   // gradient wave: v rows, B_yv, B_ysa; set-up wave: dy rows, C_dyv, C_dysa
    Split8 cs0, cs1;               // gradient wave: sa rows; set-up wave: dSA rows
    f32x4 lw4;
    {
      Rc = Split4{tr_frag(P.rows[T_RH].r, 0, 16 * kb, lane), tr_frag(P.rows[T_RL].r, 0, 16 * kb, lane)};
      Ac = Split4{tr_frag(P.rows[T_AH].r, 0, 16 * kb, lane), tr_frag(P.rows[T_AL].r, 0, 16 * kb, lane)};
      Kc = Split4{tr_frag(P.rows[T_KH].r, 0, 16 * kb, lane), tr_frag(P.rows[T_KL].r, 0, 16 * kb, lane)};
      Bc = Split4{tr_frag(P.rows[T_BH].r, 0, 16 * kb, lane), tr_frag(P.rows[T_BL].r, 0, 16 * kb, lane)};
#pragma unroll
      for (int m = 0; m < 2; ++m)
        Db[m] = Split8{tr_frag32(L.xds[0], m, 16 * kb, lane), tr_frag32(L.xds[1], m, 16 * kb, lane)};
      g4 = *reinterpret_cast<const f32x4*>(&P.gT[ki][4 * qd]);
      if (grad) {
        cv0 = row_frag(stg[S_V].r, t, 0, qd);
        cv1 = row_frag(stg[S_V].r, t, 1, qd);
        cs0 = row_pair(stg[S_SAH].r, stg[S_SAL].r, t, 0, qd);
        cs1 = row_pair(stg[S_SAH].r, stg[S_SAL].r, t, 1, qd);
        f_b0 = L.frag[G_BYV][lane];
        f_b1 = L.frag[G_BYSA][lane];
      } else {
        cv0 = row_frag(stg[S_DY].r, t, 0, qd);
        cv1 = row_frag(stg[S_DY].r, t, 1, qd);
        cs0 = Split8{dsa_frag(0, 0), dsa_frag(1, 0)};
        cs1 = Split8{dsa_frag(0, 1), dsa_frag(1, 1)};
        f_b0 = L.frag[G_CDYV][lane];
        f_b1 = L.frag[G_CDYSA][lane];
        lw4 = *reinterpret_cast<const f32x4*>(&P.lwT[ki][4 * qd]);
      }
    }
    lds_barrier();

    // ================= phase C: key-indexed gradients of key tile kb = wq,
    // result layout rows = step 4 qd + r, column = key ki; the gradient wave
    // forms dK and dB, the set-up wave dR, dA and the decay gradient's parts
    {
      const f32x4 z = {0.f, 0.f, 0.f, 0.f};
      float epart = 0.f;
      f32x4 f, suf;
      if (grad) {
        const bf16x8 v0 = cv0, v1 = cv1;
        const Split8 s0f = cs0, s1f = cs1;
        const bf16x8 f_byv = f_b0, f_bysa = f_b1;
        const bf16x8 f_bsav = L.frag[G_BSAV][lane], f_bsasa = L.frag[G_BSASA][lane];
        __builtin_amdgcn_sched_barrier(0);
        // V dS' (= d k- gamma_L) and SA dS' (= d b- gamma_L)
        f32x4 x1 = mma32(v0, Db[0].lo, z);
        x1 = mma32(v1, Db[1].lo, x1);
        x1 = mma32(v0, Db[0].hi, x1);
        x1 = mma32(v1, Db[1].hi, x1);
        f32x4 x2 = mma32x3(s0f, Db[0], z);
        x2 = mma32x3(s1f, Db[1], x2);
        f32x4 dk = mma_s3(f_byv, Rc, x1);
        dk = mma_s3(f_bsav, Ac, dk);
        f32x4 dbv = mma_s3(f_bysa, Rc, x2);
        dbv = mma_s3(f_bsasa, Ac, dbv);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float kf = hi_lo(Kc.hi, Kc.lo, r), bf = hi_lo(Bc.hi, Bc.lo, r);
          // sum over the chunk's steps of K~ o V dS' + B~ o SA dS'
          epart += kf * x1[r] + bf * x2[r];
          // this wave's part of dL/dg, before the decay factors: K~ o dk' + B~ o db'
          f[r] = kf * dk[r] + bf * dbv[r];
          const float gin = exp2_f(-g4[r]);
          out_at(outs[O_DK], 4 * qd + r, ki) = __builtin_bit_cast(bf16_t, (__bf16)(dk[r] * gin));
          out_at(outs[O_DB], 4 * qd + r, ki) = __builtin_bit_cast(bf16_t, (__bf16)(dbv[r] * gin));
        }
      } else {
        // start state as B operand (k = value j, column = key ki), split
        f32x4 S0v[2][2];
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          if constexpr (kFull || kLong) {
            S0v[m][0] = S0row[m][0];
            S0v[m][1] = S0row[m][1];
          } else {
            S0v[m][0] = *reinterpret_cast<const f32x4*>(&s0r[ki][32 * m + 4 * qd]);
            S0v[m][1] = *reinterpret_cast<const f32x4*>(&s0r[ki][32 * m + 16 + 4 * qd]);
          }
        }
        const bf16x8 y0 = cv0, y1 = cv1;
        const Split8 q0 = cs0, q1 = cs1;
        const bf16x8 f_cdyv = f_b0, f_cdysa = f_b1;
        const bf16x8 f_cdsav = L.frag[G_CDSAV][lane], f_cdsasa = L.frag[G_CDSASA][lane];
        __builtin_amdgcn_sched_barrier(0);
        Split8 S0b[2];
#pragma unroll
        for (int m = 0; m < 2; ++m) S0b[m] = split8(S0v[m][0], S0v[m][1]);
        // dY S0 and dSA S0
        f32x4 dr = mma32(y0, S0b[0].lo, z);
        dr = mma32(y1, S0b[1].lo, dr);
        dr = mma32(y0, S0b[0].hi, dr);
        dr = mma32(y1, S0b[1].hi, dr);
        dr = mma_s3(f_cdyv, Kc, dr);
        dr = mma_s3(f_cdysa, Bc, dr);
        f32x4 da = mma32x3(q0, S0b[0], z);
        da = mma32x3(q1, S0b[1], da);
        da = mma_s3(f_cdsav, Kc, da);
        da = mma_s3(f_cdsasa, Bc, da);
        // sum over this lane's 16 values j of S0 o dS' (S0 and dS' hold the
        // same j per element)
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
          for (int e = 0; e < 8; e += 2) {
            const bf16x2 sh = {S0b[m].hi[e], S0b[m].hi[e + 1]}, sl = {S0b[m].lo[e], S0b[m].lo[e + 1]};
            const bf16x2 dh = {Db[m].hi[e], Db[m].hi[e + 1]}, dl = {Db[m].lo[e], Db[m].lo[e + 1]};
            epart = __builtin_amdgcn_fdot2_f32_bf16(sh, dh, epart, false);
            epart = __builtin_amdgcn_fdot2_f32_bf16(sh, dl, epart, false);
            epart = __builtin_amdgcn_fdot2_f32_bf16(sl, dh, epart, false);
          }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float rf = hi_lo(Rc.hi, Rc.lo, r), af = hi_lo(Ac.hi, Ac.lo, r);
          const float ad = af * da[r];
          // this wave's part of dL/dg before the decay factors: R^ o dr' + A^ o da'
          f[r] = rf * dr[r] + ad;
          carry[r] = -ad;
          sig[r] = lw4[r] * kSigFromLw2;
          const float gam = exp2_f(g4[r]), gpv = exp2_f(g4[r] - lw4[r]);
          out_at(outs[O_DR], 4 * qd + r, ki) = __builtin_bit_cast(bf16_t, (__bf16)(dr[r] * gam));
          out_at(outs[O_DA], 4 * qd + r, ki) = __builtin_bit_cast(bf16_t, (__bf16)(da[r] * gpv));
        }
      }
      // suffix sums over the chunk's steps: in-lane over r, then over quads
      suf[3] = f[3];
      suf[2] = f[2] + suf[3];
      suf[1] = f[1] + suf[2];
      suf[0] = f[0] + suf[1];
      const float above = rows_after(suf[0], qd), etot = rows_total(epart);
      // dlw = (R^ o dr' + A^ o da' suffix) - (K~ o dk' + B~ o db' suffix)
      //       - a da + E: the gradient wave leaves its part, the set-up wave
      //       keeps its own and combines after the next barrier
      if (grad) {
        L.kx[kb][lane] = f32x4{suf[0] + above - etot, suf[1] + above - etot,
                               suf[2] + above - etot, suf[3] + above - etot};
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) carry[r] += suf[r] + above + etot;
      }
    }
  };
  for (int c = last; c >= 1; --c) run_chunk(c, std::true_type{});
  run_chunk(0, std::false_type{});

  lds_barrier();
  if (!grad) finish(0);
  lds_barrier();
  if (!grad) flush(0);
  if (grad && p.ds0) {
#pragma unroll
    for (int ib = 0; ib < 4; ++ib)
      *reinterpret_cast<f32x4*>(p.ds0 + bh * (kHead * kHead) + jcol * kHead + 16 * ib + 4 * qd) = dS[ib];
  }
}

}  // namespace

bool chunk_backward_supported(const BackwardDesc& d) {
  return d.dtype == Dtype::BF16 && d.C >= kL && d.C % kL == 0 && d.T % d.C == 0 && d.T > 0;
}

hipError_t launch_backward_chunked(const BackwardDesc& d, hipStream_t stream) {
  BwdChunkParams p;
  p.in[I_X] = static_cast<const bf16_t*>(d.w);
  p.in[I_R] = static_cast<const bf16_t*>(d.r);
  p.in[I_K] = static_cast<const bf16_t*>(d.k);
  p.in[I_A] = static_cast<const bf16_t*>(d.a);
  p.in[I_B] = static_cast<const bf16_t*>(d.b);
  p.in[I_V] = static_cast<const bf16_t*>(d.v);
  p.in[I_DY] = static_cast<const bf16_t*>(d.dy);
  p.ckpt = d.ckpt;
  p.sa = d.sa;
  p.dsT = d.dsT;
  p.dw = static_cast<bf16_t*>(d.dw);
  p.dr = static_cast<bf16_t*>(d.dr);
  p.dk = static_cast<bf16_t*>(d.dk);
  p.dv = static_cast<bf16_t*>(d.dv);
  p.da = static_cast<bf16_t*>(d.da);
  p.db = static_cast<bf16_t*>(d.db);
  p.ds0 = d.ds0;
  p.T = d.T;
  p.H = d.H;
  p.C = d.C;
  const dim3 grid(d.H, d.B, 1), block(kBlock, 1, 1);
  if (d.C == kL)
    hipLaunchKernelGGL(wkv7_bwd_chunk_kernel<false>, grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL(wkv7_bwd_chunk_kernel<true>, grid, block, 0, stream, p);
  return hipGetLastError();
}

}  // namespace wkv7
