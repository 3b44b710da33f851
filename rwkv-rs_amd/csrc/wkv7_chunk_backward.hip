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
// previous checkpoint.
//
// Work layout: one workgroup of four waves per (batch, head), chunks in
// reverse order, the next chunk's inputs loaded into registers meanwhile. Per
// chunk: (1) wave w computes decays and the split A^, R^, K~, B~ rows for keys
// 16w..16w+15; (2) wave w computes one of the four step-by-step products of
// decayed vectors; (3) wave 0 forms P by substitution while the others form
// the step-by-step products of the raw inputs; (4) wave w carries the state
// gradient for value columns 16w..16w+15 and writes dV; (5) the products with
// dSA; (6) wave w computes the key-indexed gradients for keys 16w..16w+15.
#include "wkv7_chunk.hpp"
#include "wkv7_launch.hpp"

namespace wkv7 {
namespace {

using namespace chunk;

constexpr int kWaves = 4;
constexpr int kBlock = 64 * kWaves;
enum { I_X, I_R, I_K, I_A, I_B, I_V, I_DY, I_COUNT };          // staged bf16 rows
enum { T_AH, T_AL, T_RH, T_RL, T_KH, T_KL, T_BH, T_BL, T_COUNT };   // decayed rows, hi/lo
enum { F_AKT, F_RBT, F_RKT, F_PT, F_BYV, F_CDYV, F_BYSA, F_CDYSA, F_BSAV, F_CDSAV,
       F_BSASA, F_CDSASA, F_COUNT };                             // stacked 16x16 operands
enum { O_DV, O_DK, O_DB, O_DR, O_DA, O_DW, O_COUNT };          // staged gradient tiles
constexpr int kOutRounds = O_COUNT * kL * 8 / (64 * 4);            // 16-byte stores per thread
constexpr int kBf16Pieces = I_COUNT * kL * 8;                    // 16-byte pieces per chunk
constexpr int kBf16Rounds = (kBf16Pieces + kBlock - 1) / kBlock;
constexpr float kSigFromLw2 = 1.0f / (kWScale * kLog2e);        // sigmoid = lw2 * this

struct BwdLds {
  bf16_t stg[2][I_COUNT][kL][64];   // raw rows of a chunk, double-buffered
  float sast[2][kL][64];            // removal_state rows, 16-byte pieces rotated by row
  bf16_t rows[T_COUNT][kL][64];     // decayed rows
  float gT[64][kL + 4];             // log2 prefix decay, [key][step]
  float lwT[64][kL + 4];            // log2 step decay, [key][step]
  float gl[64];                     // gamma_L
  bf16x8 frag[F_COUNT][64];         // 16x16 step-by-step operands, stacked (hi | lo)
  float amat[kL][kL];               // A_ab transposed, [s][t], for the substitution
  bf16_t xds[2][64][64];            // dS' hi/lo, [value j][key i]
  bf16_t xdsa[2][64][kL];           // dSA hi/lo, [value j][step t]
  float s0r[64][68];                // chunk 0's rebuilt start state, [key i][value j]
  float red[kWaves][2][4][16];      // cross-quad scratch of the key-gradient waves
  bf16_t outs[O_COUNT][kL][64];     // a chunk's bf16 gradients, written out as whole rows
};

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
};

__device__ __forceinline__ float sa_at(const float (*rows)[64], int t, int c) {
  return rows[t][4 * (((c >> 2) + t) & 15) + (c & 3)];
}
__device__ __forceinline__ f32x4 sa_read4(const float (*rows)[64], int t, int c) {
  return *reinterpret_cast<const f32x4*>(&rows[t][4 * (((c >> 2) + t) & 15)]);
}
// x32 fragment of the lane's removal_state row, split
__device__ __forceinline__ Split8 sa_frag(const float (*rows)[64], int t, int m, int qd) {
  return split8(sa_read4(rows, t, 32 * m + 4 * qd), sa_read4(rows, t, 32 * m + 16 + 4 * qd));
}
__device__ __forceinline__ f32x4 widen4(bf16x4 x) { return __builtin_convertvector(x, f32x4); }
__device__ __forceinline__ bf16x8 stack_f(f32x4 x) { return stack(split4(x)); }
// 16x16 product of two row fragment pairs over the 64 columns (k = column)
__device__ __forceinline__ f32x4 gram_x3(const Split8 (&a)[2], const Split8 (&b)[2]) {
  f32x4 c = {0.f, 0.f, 0.f, 0.f};
  c = mma32x3(a[0], b[0], c);
  return mma32x3(a[1], b[1], c);
}

__global__ __launch_bounds__(kBlock, 1) void wkv7_bwd_chunk_kernel(const BwdChunkParams p) {
  __shared__ BwdLds L;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
  const int t = lane & 15, qd = lane >> 4;
  const int h = blockIdx.x, b = blockIdx.y, H = p.H, T = p.T;
  const int64_t bh = (int64_t)b * H + h;
  const int64_t tstride = (int64_t)H * kHead;
  const int64_t tok0 = ((int64_t)b * T * H + h) * kHead;
  const int nchunks = T / kL;
  const float* const ckbh = p.ckpt + bh * nchunks * (kHead * kHead);

  // ---- staging of chunk c: thread tid moves 16-byte pieces, through
  // registers (loaded early, written to the free LDS buffer at the chunk's
  // end). bf16 rows as rotated pieces (piece p = 256 k + tid is row p / 8,
  // slot p % 8), removal_state rows as pieces rotated over 16 slots.
  struct Pre { uint4 v[kBf16Rounds + 1]; };
  // piece 256 k + tid lies in row (256 k + tid) / 8 of input 2 k + wave / 2:
  // the input index is wave-uniform, so its pointer stays in scalar registers
  auto fetch = [&](int c) {
    Pre pr;
#pragma unroll
    for (int k = 0; k < kBf16Rounds; ++k) {
      const int pc = kBlock * k + tid;
      pr.v[k] = make_uint4(0, 0, 0, 0);
      if (kBlock * k + 64 * wave < kBf16Pieces) {
        const int vec = 2 * k + (wave >> 1);
        const int slot = pc & 7, st = (pc >> 3) & 15;
        pr.v[k] = *reinterpret_cast<const uint4*>(
            p.in[vec] + tok0 + (int64_t)(kL * c + st) * tstride + 8 * ((slot - st) & 7));
      }
    }
    const int st = tid >> 4, slot = tid & 15;
    pr.v[kBf16Rounds] = *reinterpret_cast<const uint4*>(
        p.sa + tok0 + (int64_t)(kL * c + st) * tstride + 4 * ((slot - st) & 15));
    return pr;
  };
  auto stage_in = [&](const Pre pr, int sb) {
#pragma unroll
    for (int k = 0; k < kBf16Rounds; ++k) {
      const int pc = kBlock * k + tid;
      if (kBlock * k + 64 * wave < kBf16Pieces) reinterpret_cast<uint4*>(&L.stg[sb][0][0][0])[pc] = pr.v[k];
    }
    reinterpret_cast<uint4*>(&L.sast[sb][0][0])[tid] = pr.v[kBf16Rounds];
  };

  // ---- state gradient: value tile jb = wave, key tiles ib, result layout
  // (rows = key i = 16 ib + 4 qd + r, columns = value j = 16 jb + t)
  const int jb = wave, jcol = 16 * jb + t;
  f32x4 dS[4];
#pragma unroll
  for (int ib = 0; ib < 4; ++ib) {
    if (p.dsT)
      dS[ib] = *reinterpret_cast<const f32x4*>(p.dsT + bh * (kHead * kHead) + jcol * kHead + 16 * ib + 4 * qd);
    else
      dS[ib] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const int ki = 16 * wave + t;   // key of the lane in the key-gradient stage (column of its tile)

  // start state S0 of chunk c (the checkpoint of chunk c - 1) as the rows
  // [key ki][value 32 m + 4 qd .., + 16 ..] of the key stage, loaded one chunk
  // ahead, after the staging loads
  f32x4 S0row[2][2], S0row_n[2][2];
  auto load_s0 = [&](int c, f32x4 (&rowv)[2][2]) {
    if (c > 0) {
      const float* ck = ckbh + (int64_t)(c - 1) * (kHead * kHead);
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        rowv[m][0] = *reinterpret_cast<const f32x4*>(ck + ki * kHead + 32 * m + 4 * qd);
        rowv[m][1] = *reinterpret_cast<const f32x4*>(ck + ki * kHead + 32 * m + 16 + 4 * qd);
      }
    }
  };

  // the staged gradient tiles of chunk cc to memory: thread tid writes
  // 16-byte pieces p = 256 k + tid (tile p / 128, row (p / 8) % 16)
  bf16_t* const outp[O_COUNT] = {p.dv, p.dk, p.db, p.dr, p.da, p.dw};
  auto flush = [&](int cc) {
#pragma unroll
    for (int k = 0; k < kOutRounds; ++k) {
      const int pc = kBlock * k + tid, tile = pc >> 7, row = (pc >> 3) & 15, piece = pc & 7;
      const uint4 v = *reinterpret_cast<const uint4*>(&L.outs[tile][row][8 * piece]);
      *reinterpret_cast<uint4*>(outp[tile] + tok0 + (int64_t)(kL * cc + row) * tstride + 8 * piece) = v;
    }
  };

  if (nchunks > 0) stage_in(fetch(nchunks - 1), (nchunks - 1) & 1);
  Pre pre;
  load_s0(nchunks - 1, S0row);
  for (int c = nchunks - 1; c >= 0; --c) {
    const int sb = c & 1;
    const bf16_t (*const stg)[kL][64] = L.stg[sb];
    const float (*const sast)[64] = L.sast[sb];
    lds_barrier();
    if (c < nchunks - 1) flush(c + 1);   // gradients of the previous chunk

    // ================= (1) decays and decayed rows, keys 16 wave .. + 15
    {
      const int c0 = 16 * wave + 4 * qd;
      // plain float arrays around the cross-lane (DPP) operations: this
      // compiler folds DPP builtins whose source is an element of an
      // ext_vector value into a single one (all elements get element 0's)
      const uint2 xr = *reinterpret_cast<const uint2*>(tile_at(stg[I_X], t, c0));
      const float xs[4] = {__uint_as_float(xr.x << 16), __uint_as_float(xr.x & 0xffff0000u),
                           __uint_as_float(xr.y << 16), __uint_as_float(xr.y & 0xffff0000u)};
      float g2[4], lw2[4], gam[4], gin[4], gpv[4], gL[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        lw2[e] = log2_decay(xs[e]);
        g2[e] = row_scan16(lw2[e]);
        gam[e] = exp2_f(g2[e]);
        gin[e] = exp2_f(-g2[e]);
        gpv[e] = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
            __builtin_bit_cast(int, 1.0f), __builtin_bit_cast(int, gam[e]), 0x111, 0xf, 0xf, false));
        gL[e] = row_last16(gam[e]);
      }
      const f32x4 gamv = {gam[0], gam[1], gam[2], gam[3]};
      const f32x4 ginv = {gin[0], gin[1], gin[2], gin[3]};
      const f32x4 gpvv = {gpv[0], gpv[1], gpv[2], gpv[3]};
      const Split4 ah = split4(widen4(read4(stg[I_A], t, c0)) * gpvv);
      const Split4 rh = split4(widen4(read4(stg[I_R], t, c0)) * gamv);
      const Split4 kt = split4(widen4(read4(stg[I_K], t, c0)) * ginv);
      const Split4 bt = split4(widen4(read4(stg[I_B], t, c0)) * ginv);
      write4(L.rows[T_AH], t, c0, ah.hi);
      write4(L.rows[T_AL], t, c0, ah.lo);
      write4(L.rows[T_RH], t, c0, rh.hi);
      write4(L.rows[T_RL], t, c0, rh.lo);
      write4(L.rows[T_KH], t, c0, kt.hi);
      write4(L.rows[T_KL], t, c0, kt.lo);
      write4(L.rows[T_BH], t, c0, bt.hi);
      write4(L.rows[T_BL], t, c0, bt.lo);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        L.gT[c0 + e][t] = g2[e];
        L.lwT[c0 + e][t] = lw2[e];
      }
      if (t == 0) *reinterpret_cast<f32x4*>(&L.gl[c0]) = f32x4{gL[0], gL[1], gL[2], gL[3]};
    }
    lds_barrier();
    if (c > 0) {
      pre = fetch(c - 1);
      load_s0(c - 1, S0row_n);
    }

    // ================= (2) step-by-step products of decayed rows, one per wave
    {
      auto rowpair = [&](int th, int tl, Split8 (&o)[2]) {
#pragma unroll
        for (int m = 0; m < 2; ++m)
          o[m] = Split8{row_frag(L.rows[th], t, m, qd), row_frag(L.rows[tl], t, m, qd)};
      };
      Split8 X[2], Y[2];
      if (wave == 0) {          // A_ab for the substitution, stored by columns
        rowpair(T_AH, T_AL, X);
        rowpair(T_BH, T_BL, Y);
        f32x4 d = gram_x3(X, Y);   // [t'][s] = a^_t' . b~_s, lane column s = t
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (!(t < 4 * qd + r)) d[r] = 0.f;
        *reinterpret_cast<f32x4*>(&L.amat[t][4 * qd]) = d;
      } else {
        const int ta = wave == 1 ? T_AH : T_RH;
        const int tb = wave == 2 ? T_BH : T_KH;
        rowpair(ta, ta + 1, X);
        rowpair(tb, tb + 1, Y);
        f32x4 d = gram_x3(X, Y);   // [t'][s'] = x_t' . y_s', the A operand of the transpose
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tp = 4 * qd + r;
          if (wave == 1 ? !(t < tp) : !(t <= tp)) d[r] = 0.f;
        }
        L.frag[wave == 1 ? F_AKT : wave == 2 ? F_RBT : F_RKT][lane] = stack_f(d);
      }
    }
    lds_barrier();

    // ================= (3) P by substitution (wave 0); raw step products
    if (wave == 0) {
      // column t of P = (I - A_ab)^-1, column-oriented: once pc[s] is final,
      // it updates every later row, so the dependent chain is 15 FMAs long
      float pc[kL];
#pragma unroll
      for (int tt = 0; tt < kL; ++tt) pc[tt] = (tt == t) ? 1.0f : 0.0f;
#pragma unroll
      for (int s = 0; s < kL - 1; ++s) {
#pragma unroll
        for (int t4 = (s + 1) & ~3; t4 < kL; t4 += 4) {
          const f32x4 acol = *reinterpret_cast<const f32x4*>(&L.amat[s][t4]);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (t4 + e > s) pc[t4 + e] += acol[e] * pc[s];
        }
      }
      // P^T as an A operand: lane l holds P[4 qd + e][l % 16], this lane's column
      f32x4 pt;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        pt[e] = qd == 0 ? pc[e] : qd == 1 ? pc[4 + e] : qd == 2 ? pc[8 + e] : pc[12 + e];
      L.frag[F_PT][lane] = stack_f(pt);
    } else {
      const bf16x8 v0 = row_frag(stg[I_V], t, 0, qd), v1 = row_frag(stg[I_V], t, 1, qd);
      const bf16x8 y0 = row_frag(stg[I_DY], t, 0, qd), y1 = row_frag(stg[I_DY], t, 1, qd);
      f32x4 z = {0.f, 0.f, 0.f, 0.f};
      if (wave == 1) {
        // B_yv^T[s][t] = dy_s . v_t, kept where s >= t; C_dyv^T[s][t] = v_s . dy_t, s <= t
        f32x4 d = mma32(y1, v1, mma32(y0, v0, z));
        f32x4 e = mma32(v1, y1, mma32(v0, y0, z));
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (!(4 * qd + r >= t)) d[r] = 0.f;
          if (!(4 * qd + r <= t)) e[r] = 0.f;
        }
        L.frag[F_BYV][lane] = stack_f(d);
        L.frag[F_CDYV][lane] = stack_f(e);
      } else {
        const Split8 s0f = sa_frag(sast, t, 0, qd), s1f = sa_frag(sast, t, 1, qd);
        f32x4 d;
        if (wave == 2) {   // B_ysa^T[s][t] = dy_s . sa_t, s >= t
          d = mma32(y0, s0f.lo, z);
          d = mma32(y1, s1f.lo, d);
          d = mma32(y0, s0f.hi, d);
          d = mma32(y1, s1f.hi, d);
        } else {           // C_dysa^T[s][t] = sa_s . dy_t, s <= t
          d = mma32(s0f.lo, y0, z);
          d = mma32(s1f.lo, y1, d);
          d = mma32(s0f.hi, y0, d);
          d = mma32(s1f.hi, y1, d);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (wave == 2 ? !(4 * qd + r >= t) : !(4 * qd + r <= t)) d[r] = 0.f;
        L.frag[wave == 2 ? F_BYSA : F_CDYSA][lane] = stack_f(d);
      }
    }
    lds_barrier();

    // ================= (4) state gradient, value tile jb
    if (c == 0) {
      // rebuild S0 by reversing the chunk's 16 steps from its checkpoint
      // (kernel.rs:239-246): S_{t-1} = (S_t - v_t k_t^T - sa_t b_t^T) / w~_t
      const float* ck = ckbh;
      f32x4 S0t[4];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int r = 0; r < 4; ++r) S0t[ib][r] = ck[(16 * ib + 4 * qd + r) * kHead + jcol];
      for (int tt = kL - 1; tt >= 0; --tt) {
        const float vj = __uint_as_float((uint32_t)stg[I_V][tt][8 * (((jcol >> 3) + tt) & 7) + (jcol & 7)] << 16);
        const float sj = sa_at(sast, tt, jcol);
#pragma unroll
        for (int ib = 0; ib < 4; ++ib) {
          const f32x4 kv = widen4(read4(stg[I_K], tt, 16 * ib + 4 * qd));
          const f32x4 bv = widen4(read4(stg[I_B], tt, 16 * ib + 4 * qd));
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float winv = exp2_f(-L.lwT[16 * ib + 4 * qd + r][tt]);
            S0t[ib][r] = (S0t[ib][r] - kv[r] * vj - bv[r] * sj) * winv;
          }
        }
      }
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int r = 0; r < 4; ++r) L.s0r[16 * ib + 4 * qd + r][jcol] = S0t[ib][r];
    }
    {
      f32x4 dSp[4];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
        dSp[ib] = dS[ib] * *reinterpret_cast<const f32x4*>(&L.gl[16 * ib + 4 * qd]);
      const Split8 Sx0 = split8(dSp[0], dSp[1]), Sx1 = split8(dSp[2], dSp[3]);
      const Split8 Bt0{row_frag(L.rows[T_BH], t, 0, qd), row_frag(L.rows[T_BL], t, 0, qd)};
      const Split8 Bt1{row_frag(L.rows[T_BH], t, 1, qd), row_frag(L.rows[T_BL], t, 1, qd)};
      const Split8 Kt0{row_frag(L.rows[T_KH], t, 0, qd), row_frag(L.rows[T_KL], t, 0, qd)};
      const Split8 Kt1{row_frag(L.rows[T_KH], t, 1, qd), row_frag(L.rows[T_KL], t, 1, qd)};
      const bf16x4 dycf = tr_frag(stg[I_DY], 0, 16 * jb, lane);   // dY[s][j] (k = s)
      f32x4 z = mma32x3(Bt0, Sx0, f32x4{0.f, 0.f, 0.f, 0.f});
      z = mma32x3(Bt1, Sx1, z);
      z = mma_s2(L.frag[F_RBT][lane], dycf, z);
      const f32x4 dsa = mma_s3(L.frag[F_PT][lane], split4(z), f32x4{0.f, 0.f, 0.f, 0.f});
      const Split4 dsas = split4(dsa);
      f32x4 dv = mma32x3(Kt0, Sx0, f32x4{0.f, 0.f, 0.f, 0.f});
      dv = mma32x3(Kt1, Sx1, dv);
      dv = mma_s2(L.frag[F_RKT][lane], dycf, dv);
      dv = mma_s3(L.frag[F_AKT][lane], dsas, dv);
#pragma unroll
      for (int r = 0; r < 4; ++r) L.outs[O_DV][4 * qd + r][jcol] = __builtin_bit_cast(bf16_t, (__bf16)dv[r]);
      // carried gradient dS0^T = dS'^T + R^^T dY + A^^T dSA
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
        const bf16x8 rT = cat8(tr_frag(L.rows[T_RH], 0, 16 * ib, lane), tr_frag(L.rows[T_RL], 0, 16 * ib, lane));
        const bf16x8 aT = cat8(tr_frag(L.rows[T_AH], 0, 16 * ib, lane), tr_frag(L.rows[T_AL], 0, 16 * ib, lane));
        f32x4 acc = mma_s2(rT, dycf, dSp[ib]);
        dS[ib] = mma_s3(aT, dsas, acc);
      }
      // exchange for the key stage: dS' as [value j][key i], dSA as [j][step]
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const Split8& sx = m ? Sx1 : Sx0;
          write4(L.xds[0], jcol, 32 * m + 16 * hh + 4 * qd, half_of(sx.hi, hh));
          write4(L.xds[1], jcol, 32 * m + 16 * hh + 4 * qd, half_of(sx.lo, hh));
        }
      *reinterpret_cast<bf16x4*>(&L.xdsa[0][jcol][4 * qd]) = dsas.hi;
      *reinterpret_cast<bf16x4*>(&L.xdsa[1][jcol][4 * qd]) = dsas.lo;
    }
    lds_barrier();

    // ================= (5) step products with dSA
    // dSA as row fragments (row = step t, k = value), from the [j][t] tiles
    auto dsa_frag = [&](int hl, int m) {
      return cat8(read_tr16(&L.xdsa[hl][32 * m + 4 * qd + (t >> 2)][4 * (t & 3)]) ,
                  read_tr16(&L.xdsa[hl][32 * m + 16 + 4 * qd + (t >> 2)][4 * (t & 3)]));
    };
    if (wave < 3) {
      const Split8 q0{dsa_frag(0, 0), dsa_frag(1, 0)}, q1{dsa_frag(0, 1), dsa_frag(1, 1)};
      f32x4 z = {0.f, 0.f, 0.f, 0.f};
      if (wave == 0) {
        const bf16x8 v0 = row_frag(stg[I_V], t, 0, qd), v1 = row_frag(stg[I_V], t, 1, qd);
        // B_sav^T[s][t] = dsa_s . v_t, s > t; C_dsav^T[s][t] = v_s . dsa_t, s < t
        f32x4 d = mma32(q0.lo, v0, z);
        d = mma32(q1.lo, v1, d);
        d = mma32(q0.hi, v0, d);
        d = mma32(q1.hi, v1, d);
        f32x4 e = mma32(v0, q0.lo, z);
        e = mma32(v1, q1.lo, e);
        e = mma32(v0, q0.hi, e);
        e = mma32(v1, q1.hi, e);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (!(4 * qd + r > t)) d[r] = 0.f;
          if (!(4 * qd + r < t)) e[r] = 0.f;
        }
        L.frag[F_BSAV][lane] = stack_f(d);
        L.frag[F_CDSAV][lane] = stack_f(e);
      } else {
        const Split8 s0f = sa_frag(sast, t, 0, qd), s1f = sa_frag(sast, t, 1, qd);
        f32x4 d;
        if (wave == 1) {   // B_sasa^T[s][t] = dsa_s . sa_t, s > t
          d = mma32x3(q0, s0f, z);
          d = mma32x3(q1, s1f, d);
        } else {           // C_dsasa^T[s][t] = sa_s . dsa_t, s < t
          d = mma32x3(s0f, q0, z);
          d = mma32x3(s1f, q1, d);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (wave == 1 ? !(4 * qd + r > t) : !(4 * qd + r < t)) d[r] = 0.f;
        L.frag[wave == 1 ? F_BSASA : F_CDSASA][lane] = stack_f(d);
      }
    }
    lds_barrier();

    // ================= (6) key-indexed gradients, keys 16 wave .. + 15
    {
      const int kb = wave;   // key tile; result layout rows = step 4 qd + r, column = key ki
      // decayed rows as B operands (k = step, column = key), split
      const Split4 Rc{tr_frag(L.rows[T_RH], 0, 16 * kb, lane), tr_frag(L.rows[T_RL], 0, 16 * kb, lane)};
      const Split4 Ac{tr_frag(L.rows[T_AH], 0, 16 * kb, lane), tr_frag(L.rows[T_AL], 0, 16 * kb, lane)};
      const Split4 Kc{tr_frag(L.rows[T_KH], 0, 16 * kb, lane), tr_frag(L.rows[T_KL], 0, 16 * kb, lane)};
      const Split4 Bc{tr_frag(L.rows[T_BH], 0, 16 * kb, lane), tr_frag(L.rows[T_BL], 0, 16 * kb, lane)};
      // start state as B operand (k = value j, column = key ki), split
      Split8 S0b[2];
      if (c > 0) {
#pragma unroll
        for (int m = 0; m < 2; ++m) S0b[m] = split8(S0row[m][0], S0row[m][1]);
      } else {
#pragma unroll
        for (int m = 0; m < 2; ++m)
          S0b[m] = split8(*reinterpret_cast<const f32x4*>(&L.s0r[ki][32 * m + 4 * qd]),
                          *reinterpret_cast<const f32x4*>(&L.s0r[ki][32 * m + 16 + 4 * qd]));
      }
      const f32x4 z = {0.f, 0.f, 0.f, 0.f};
      // dS' as B operand (k = value j, column = key ki)
      Split8 Db[2];
#pragma unroll
      for (int m = 0; m < 2; ++m)
        Db[m] = Split8{tr_frag32(L.xds[0], m, 16 * kb, lane), tr_frag32(L.xds[1], m, 16 * kb, lane)};
      const bf16x8 v0 = row_frag(stg[I_V], t, 0, qd), v1 = row_frag(stg[I_V], t, 1, qd);
      const bf16x8 y0 = row_frag(stg[I_DY], t, 0, qd), y1 = row_frag(stg[I_DY], t, 1, qd);
      const Split8 s0f = sa_frag(sast, t, 0, qd), s1f = sa_frag(sast, t, 1, qd);
      const Split8 q0{dsa_frag(0, 0), dsa_frag(1, 0)}, q1{dsa_frag(0, 1), dsa_frag(1, 1)};

      // V dS' (= d k- gamma_L) and SA dS' (= d b- gamma_L)
      f32x4 x1 = mma32(v0, Db[0].lo, z);
      x1 = mma32(v1, Db[1].lo, x1);
      x1 = mma32(v0, Db[0].hi, x1);
      x1 = mma32(v1, Db[1].hi, x1);
      f32x4 x2 = mma32x3(s0f, Db[0], z);
      x2 = mma32x3(s1f, Db[1], x2);
      // sum over the chunk's steps of K~ o V dS' + B~ o SA dS', and over this
      // lane's 16 values j of S0 o dS' (S0 and dS' hold the same j per element)
      float epart = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        epart += ((float)Kc.hi[r] + (float)Kc.lo[r]) * x1[r] + ((float)Bc.hi[r] + (float)Bc.lo[r]) * x2[r];
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
      f32x4 dk = mma_s3(L.frag[F_BYV][lane], Rc, x1);
      dk = mma_s3(L.frag[F_BSAV][lane], Ac, dk);
      f32x4 dbv = mma_s3(L.frag[F_BYSA][lane], Rc, x2);
      dbv = mma_s3(L.frag[F_BSASA][lane], Ac, dbv);
      // dY S0 and dSA S0
      f32x4 dr = mma32(y0, S0b[0].lo, z);
      dr = mma32(y1, S0b[1].lo, dr);
      dr = mma32(y0, S0b[0].hi, dr);
      dr = mma32(y1, S0b[1].hi, dr);
      dr = mma_s3(L.frag[F_CDYV][lane], Kc, dr);
      dr = mma_s3(L.frag[F_CDYSA][lane], Bc, dr);
      f32x4 da = mma32x3(q0, S0b[0], z);
      da = mma32x3(q1, S0b[1], da);
      da = mma_s3(L.frag[F_CDSAV][lane], Kc, da);
      da = mma_s3(L.frag[F_CDSASA][lane], Bc, da);

      // decay factors at (step 4 qd + r, key ki)
      const f32x4 g4 = *reinterpret_cast<const f32x4*>(&L.gT[ki][4 * qd]);
      const f32x4 lw4 = *reinterpret_cast<const f32x4*>(&L.lwT[ki][4 * qd]);
      const f32x4 rv = widen4(tr_frag(stg[I_R], 0, 16 * kb, lane));
      const f32x4 kv = widen4(tr_frag(stg[I_K], 0, 16 * kb, lane));
      const f32x4 bv = widen4(tr_frag(stg[I_B], 0, 16 * kb, lane));
      const f32x4 av = widen4(tr_frag(stg[I_A], 0, 16 * kb, lane));
      f32x4 f, ad, sig;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float gam = exp2_f(g4[r]), gin = exp2_f(-g4[r]), gpv = exp2_f(g4[r] - lw4[r]);
        dk[r] *= gin;
        dbv[r] *= gin;
        dr[r] *= gam;
        da[r] *= gpv;
        ad[r] = av[r] * da[r];
        f[r] = rv[r] * dr[r] - kv[r] * dk[r] - bv[r] * dbv[r] + ad[r];
        sig[r] = lw4[r] * kSigFromLw2;
      }
      // suffix sums over the chunk's steps: in-lane over r, then over quads
      f32x4 suf;
      suf[3] = f[3];
      suf[2] = f[2] + suf[3];
      suf[1] = f[1] + suf[2];
      suf[0] = f[0] + suf[1];
      L.red[wave][0][qd][t] = suf[0];
      L.red[wave][1][qd][t] = epart;
      wave_lds_sync();
      float above = 0.f, etot = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float fq = L.red[wave][0][q][t];
        above += q > qd ? fq : 0.f;
        etot += L.red[wave][1][q][t];
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float dlw = suf[r] + above - ad[r] + etot;
        const float dwv = dlw * kWScale * sig[r] * (1.0f - sig[r]);
        const int tr = 4 * qd + r;
        L.outs[O_DK][tr][ki] = __builtin_bit_cast(bf16_t, (__bf16)dk[r]);
        L.outs[O_DB][tr][ki] = __builtin_bit_cast(bf16_t, (__bf16)dbv[r]);
        L.outs[O_DR][tr][ki] = __builtin_bit_cast(bf16_t, (__bf16)dr[r]);
        L.outs[O_DA][tr][ki] = __builtin_bit_cast(bf16_t, (__bf16)da[r]);
        L.outs[O_DW][tr][ki] = __builtin_bit_cast(bf16_t, (__bf16)dwv);
      }
    }
    if (c > 0) stage_in(pre, sb ^ 1);   // next chunk's rows into the free buffer
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      S0row[m][0] = S0row_n[m][0];
      S0row[m][1] = S0row_n[m][1];
    }
  }

  if (nchunks > 0) {
    lds_barrier();
    flush(0);
  }
  if (p.ds0) {
#pragma unroll
    for (int ib = 0; ib < 4; ++ib)
      *reinterpret_cast<f32x4*>(p.ds0 + bh * (kHead * kHead) + jcol * kHead + 16 * ib + 4 * qd) = dS[ib];
  }
}

}  // namespace

bool chunk_backward_supported(const BackwardDesc& d) {
  return d.dtype == Dtype::BF16 && d.C == kL && d.T % kL == 0 && d.T > 0;
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
  const dim3 grid(d.H, d.B, 1), block(kBlock, 1, 1);
  hipLaunchKernelGGL(wkv7_bwd_chunk_kernel, grid, block, 0, stream, p);
  return hipGetLastError();
}

}  // namespace wkv7
