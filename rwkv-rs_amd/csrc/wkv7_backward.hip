// WKV7 backward recurrence for gfx950, all six input gradients and the
// initial-state gradient in one pass.
//
// Semantics: /root/reference/crates/rwkv-nn/src/kernels/wkv7_common/kernel.rs:116-308
// (wkv7_backward_kernel), per (batch b, head h), t = T-1..0, dS = ds_T or 0:
//   if (t+1) % C == 0: S = checkpoint[t / C]           (exact reload, :210-228)
//   dr_t   = S_t^T dy_t                                             (:230-237)
//   S_{t-1} = (S_t - v k^T - sa b^T) / w~    (rebuild by reversal,  :239-246)
//   dS    += dy r^T                                                 (:248-249)
//   dw~_i  = sum_j dS[j,i] S_{t-1}[j,i];  dk = dS^T v;  db = dS^T sa (:258-265)
//   dv     = dS k;  dsa = dS b
//   dw     = W_SCALE * dw~ * w~ * sigmoid(w) * (1 - sigmoid(w))    (:267-271)
//   da     = S_{t-1}^T dsa                                          (:280-287)
//   dS     = dS diag(w~) + dsa a^T                                  (:289-296)
//   ds0    = dS after t = 0                                         (:299-307)
//
// Design. One 512-thread workgroup per (b, h). Thread tid = 16*q + L plays two
// roles on two transposed 2x4 blocks (layout and lane-relative order in
// wkv7_device.hpp; d = 0 is the thread's own row/column 2q + up, d = 1 the
// other one):
//   row role:    dSo/dSt[c] = dS[own/other row][4L+c] -> row sums dv, dsa
//   column role: Sc[c][d]  = S[4L+c][column d],
//                dSc[c][d] = dS[4L+c][column d]      -> column sums dr, dw~,
//                                                       dk, db, da
// The sixteen lanes of a DPP row (same q) span all 64 columns in the row role
// and all 64 rows in the column role, so every sum is in-lane products plus a
// DPP reduction over the row. Keeping dS twice costs 3 instructions per
// element per step; reducing the five column sums across waves instead would
// cost more. Every operand arrives as one ds_read_b128 of an LDS vector (the
// thread's four columns for the row role, its four rows for the column role)
// or of a packed per-column-pair record, consumed by plain full-rate FMAs.
// The only data exchanged between waves is dsa (64 floats, needed by the
// column role): one LDS vector and one barrier per step. dsa is the only sum
// on the step-to-step dependency chain; the twelve per-step partial sums of
// the six gradients stay in registers for 8 steps and are reduced in one
// batch.
#include "wkv7_device.hpp"
#include "wkv7_launch.hpp"

namespace wkv7 {
namespace {

// Timesteps per LDS tile: 16 for bf16 operands, 8 for fp32 ones (whose raw
// rows and staged gradients take twice the LDS). The gradient partials are
// reduced in batches of kHalf steps (96 values per lane).
template <typename Tin> constexpr int tile_len() { return sizeof(Tin) == 2 ? 16 : 8; }
constexpr int kHalf = 8;

// fp32 LDS vectors per timestep (64 entries)
enum {
  V_R = 0, V_K, V_B, V_W, V_A,   // key-indexed: row role
  V_DY, V_V, V_SA,               // value-indexed: column role
  V_DWF,                         // W_SCALE * w~ * sig * (1 - sig)
  V_DYS,                         // dy with each row pair swapped (row role, upper half);
                                 // last: it is stored 128 bytes further (see tile_mem)
  V_COUNT
};
// per-column-pair records for the column role, float4 {x[2p], x[2p+1],
// y[2p], y[2p+1]}; a second copy with each pair swapped serves the upper
// half-rows. k and b enter the column role only through the reversal
// (S - k v - b sa), so they are stored negated: the FMAs then need no source
// modifier and encode as two-operand v_fmac.
enum { P_RK = 0, P_BA, P_WI, P_COUNT };   // {r, -k}, {-b, a}, {w~, 1/w~}
// gradient outputs, in the order of the per-step partials
enum { O_DV = 0, O_DR, O_DW, O_DK, O_DB, O_DA, O_COUNT };
// raw (input dtype) operand rows as loaded from global memory
enum { R_W = 0, R_R, R_K, R_V, R_A, R_B, R_DY, R_COUNT };

__device__ __forceinline__ void unpack4(float* d, float4 x) {
  d[0] = x.x; d[1] = x.y; d[2] = x.z; d[3] = x.w;
}

template <typename Tin>
struct BwdParams {
  const Tin* in[R_COUNT];   // w, r, k, v, a, b, dy (R_* order)
  const float* ckpt;
  const float* sa;
  const float* dsT;
  Tin *dw, *dr, *dk, *dv, *da, *db;
  float* ds0;
  int T, H, C;
};

// kCkTiled: C is a multiple of the tile length, so every tile is full (T is a
// multiple of C), every checkpoint reload happens at the first step processed
// in a tile, and the checkpoint travels with that tile (loaded into LDS one
// tile ahead); the steps of a tile then form one branch-free block.
// Otherwise the last tile may be partial and reloads read global memory at
// any step.
template <typename Tin, bool kCkTiled>
__global__ __launch_bounds__(kThreads) void wkv7_bwd_kernel(BwdParams<Tin> p) {
  constexpr int kTile = tile_len<Tin>();
  constexpr int kRow = kHead * sizeof(Tin);                // bytes of one raw row
  constexpr int kRawBytes = R_COUNT * kTile * kRow + kTile * kHead * 4;
  constexpr int kParts = 2 * O_COUNT * kHalf;              // partial sums per batch
  // The swapped copies (pair records, dy) are read by the upper half-rows in
  // the same instruction as the plain ones by the lower half-rows; they are
  // placed 64 / 128 bytes off a 256-byte boundary relative to the plain data,
  // so the two sets of addresses fall into different LDS banks.
  constexpr int kPairsCopy = P_COUNT * kTile * 32 + 4;      // float4s per copy (+64 B)
  __shared__ float4 tile_mem[V_COUNT * kTile * 16 + 8];    // 20 KiB per 8 steps
  __shared__ float4 pairs_mem[2 * kPairsCopy];             // 24 KiB per 8 steps: plain, swapped
  // total for bf16 (16 steps): 40 + 48 + 12 + 32 + 18 + 2.5 KiB; fp32 (8): 20 + 24 + 12 + 32 + 16 + 2.5
  __shared__ Tin ost[O_COUNT][kTile][kHead];               // gradients in the output dtype
  __shared__ float4 ckbuf[2][kHead * kHead / 4];           // 32 KiB, by tile parity
  __shared__ float4 raw[kRawBytes / 16];                   // 18 (bf16) or 16 (fp32) KiB
  __shared__ float dsab[2][kHalf][kHead];                  // dsa of a batch, by batch parity
  __shared__ float dump[64];                               // sink of unselected lanes

  // row s of LDS vector V (V_DYS sits 128 bytes further, see above)
  static_assert(V_DYS == V_COUNT - 1, "the shifted vector must be the last one");
  auto tile = [&](int V, int s) -> float4* {
    return tile_mem + (V * kTile + s) * 16 + (V == V_DYS ? 8 : 0);
  };
  auto pairs = [&](int h, int rec, int s) -> float4* {
    return pairs_mem + h * kPairsCopy + (rec * kTile + s) * 32;
  };
  const int h = blockIdx.x, bi = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int L = tid & 15, q = tid >> 4;
  const int up = (L >> 3) & 1;
  const int ro = 2 * q + up, rt = 2 * q + 1 - up;   // own and other row / column
  // conversion: the decay of element pair 2e, 2e+1 (e = tid % 32) of
  // timesteps tid / 32 + 16u, then group sg = tid / 128 (0: r, k; 1: b, a;
  // 2: dy, v, sa; 3: none) widens elements 4pp .. 4pp+3 of timesteps
  // sl + 8u; flush: the same (sl, pp)
  const int sg = tid >> 7, sl = (tid >> 4) & 7, pp = tid & 15;

  const int T = p.T, C = p.C;
  const int64_t bh = (int64_t)bi * p.H + h;
  const int64_t tstride = (int64_t)p.H * kHead;
  const int64_t tok0 = ((int64_t)bi * T * p.H + h) * kHead;
  const int64_t nchunks = T / C;
  const float* ckpt_bh = p.ckpt + bh * nchunks * (kHead * kHead);
  auto ck_needed = [&](int t0, int nst) { return kCkTiled && ((t0 + nst) % C) == 0; };

  // Loads of one tile: 16-byte chunk c0 + lane of `raw` for c0 = wave base +
  // kThreads * j. The source of a chunk moves by a whole number of timesteps
  // from tile to tile, so its address at timestep 0 and its timestep within
  // the tile are computed once here.
  constexpr int kChunksTok = R_COUNT * kTile * kRow / 16;
  constexpr int kChunks = kRawBytes / 16;
  constexpr int kIssue = (kChunks + kThreads - 1) / kThreads;
  const char* isrc[kIssue];
  int istep[kIssue];
#pragma unroll
  for (int j = 0; j < kIssue; ++j) {
    const int c0 = tid - lane + kThreads * j, c = c0 + lane;
    if (c0 < kChunksTok) {
      const int row = c / (kRow / 16), col = c % (kRow / 16);
      istep[j] = row % kTile;
      const Tin* base = p.in[__builtin_amdgcn_readfirstlane(c0 / (kRow / 16)) / kTile];
      isrc[j] = reinterpret_cast<const char*>(base + tok0 + (int64_t)istep[j] * tstride) + 16 * col;
    } else {
      const int cc = c - kChunksTok;
      istep[j] = cc / 16;
      isrc[j] = reinterpret_cast<const char*>(p.sa + tok0 + (int64_t)istep[j] * tstride) + 16 * (cc % 16);
    }
  }
  // Issue the loads of tile [t0, t0+nst) into `raw` (and its checkpoint into
  // ckbuf[par]); they complete while another tile is computed.
  auto issue = [&](int t0, int nst, int par) {
    const int64_t shift = (int64_t)t0 * tstride * (int64_t)sizeof(Tin);   // bytes, uniform
    const int64_t shift_sa = (int64_t)t0 * tstride * 4;
#pragma unroll
    for (int j = 0; j < kIssue; ++j) {
      const int c0 = tid - lane + kThreads * j;
      if (c0 < kChunks && (kCkTiled || istep[j] < nst))
        load_lds16(isrc[j] + (c0 < kChunksTok ? shift : shift_sa), &raw[c0]);
    }
    if (ck_needed(t0, nst)) {
      const float4* src = reinterpret_cast<const float4*>(
          ckpt_bh + (int64_t)((t0 + nst) / C - 1) * (kHead * kHead));
      load_lds16(src + tid, &ckbuf[par][tid - lane]);
      load_lds16(src + kThreads + tid, &ckbuf[par][kThreads + tid - lane]);
    }
  };
  // raw tile -> fp32 operand vectors and column-pair records (plain, swapped)
  auto convert = [&](int nst) {
    const char* rb = reinterpret_cast<const char*>(raw);
#pragma unroll
    for (int u = 0; u < (kTile + 15) / 16; ++u) {   // w -> w~, 1/w~, dw factor
      const int ws_ = (tid >> 5) + 16 * u, e = tid & 31;
      if (ws_ < nst) {
        float x[2];
        if constexpr (sizeof(Tin) == 2) {
          const uint32_t b2 = reinterpret_cast<const uint32_t*>(rb + (R_W * kTile + ws_) * kRow)[e];
          x[0] = bf16_to_f32(b2 & 0xffffu);
          x[1] = bf16_to_f32(b2 >> 16);
        } else {
          const float2 f2 = reinterpret_cast<const float2*>(rb + (R_W * kTile + ws_) * kRow)[e];
          x[0] = f2.x;
          x[1] = f2.y;
        }
        float w[2], iw[2], dwf[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const float sig = sigmoid_f(x[b]);
          w[b] = decay_f(sig);
          iw[b] = 1.0f / w[b];
          dwf[b] = kWScale * w[b] * sig * (1.0f - sig);
        }
        reinterpret_cast<float2*>(tile(V_W, ws_))[e] = make_float2(w[0], w[1]);
        reinterpret_cast<float2*>(tile(V_DWF, ws_))[e] = make_float2(dwf[0], dwf[1]);
        pairs(0, P_WI, ws_)[e] = make_float4(w[0], w[1], iw[0], iw[1]);
        pairs(1, P_WI, ws_)[e] = make_float4(w[1], w[0], iw[1], iw[0]);
      }
    }
#pragma unroll
    for (int u = 0; u < kTile / 8; ++u) {
      const int st = sl + 8 * u;
      if (st >= nst) break;
      auto rawv = [&](int vec) {
        return Io<Tin>::widen(*reinterpret_cast<const typename Io<Tin>::raw*>(
            rb + (vec * kTile + st) * kRow + 4 * pp * sizeof(Tin)));
      };
      auto put_pairs = [&](int rec, float4 x, float4 y) {
        pairs(0, rec, st)[2 * pp] = make_float4(x.x, x.y, y.x, y.y);
        pairs(0, rec, st)[2 * pp + 1] = make_float4(x.z, x.w, y.z, y.w);
        pairs(1, rec, st)[2 * pp] = make_float4(x.y, x.x, y.y, y.x);
        pairs(1, rec, st)[2 * pp + 1] = make_float4(x.w, x.z, y.w, y.z);
      };
      if (sg == 0) {
        const float4 r = rawv(R_R), k = rawv(R_K);
        tile(V_R, st)[pp] = r;
        tile(V_K, st)[pp] = k;
        put_pairs(P_RK, r, make_float4(-k.x, -k.y, -k.z, -k.w));
      } else if (sg == 1) {
        const float4 b = rawv(R_B), a = rawv(R_A);
        tile(V_B, st)[pp] = b;
        tile(V_A, st)[pp] = a;
        put_pairs(P_BA, make_float4(-b.x, -b.y, -b.z, -b.w), a);
      } else if (sg == 2) {
        const float4 dy = rawv(R_DY);
        tile(V_DY, st)[pp] = dy;
        tile(V_DYS, st)[pp] = make_float4(dy.y, dy.x, dy.w, dy.z);
        tile(V_V, st)[pp] = rawv(R_V);
        tile(V_SA, st)[pp] = *reinterpret_cast<const float4*>(
            rb + R_COUNT * kTile * kRow + (st * kHead + 4 * pp) * 4);
      }
    }
  };
  // (own, other) rows of dy for the row role: 32 float2 per step row
  const float2* dyrow = reinterpret_cast<const float2*>(tile(up ? V_DYS : V_DY, 0)) + q;
  const float4* prec = pairs_mem + up * kPairsCopy + q;   // this half-row's pair records

  float dSo[4], dSt[4], Sc[4][2], dSc[4][2];
#pragma unroll
  for (int c = 0; c < 4; ++c) { Sc[c][0] = 0.0f; Sc[c][1] = 0.0f; }
  if (p.dsT) {
    const float* g0 = p.dsT + bh * (kHead * kHead);
    unpack4(dSo, *reinterpret_cast<const float4*>(g0 + ro * kHead + 4 * L));
    unpack4(dSt, *reinterpret_cast<const float4*>(g0 + rt * kHead + 4 * L));
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      dSc[c][0] = g0[(4 * L + c) * kHead + ro];
      dSc[c][1] = g0[(4 * L + c) * kHead + rt];
    }
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      dSo[c] = 0.0f; dSt[c] = 0.0f; dSc[c][0] = 0.0f; dSc[c][1] = 0.0f;
    }
  }

  // checkpoint key-rows own/other, entries 4L .. 4L+3, are Sc[0..3][0/1]
  auto reload = [&](float4 x0, float4 x1) {   // kernel.rs:210-228
    Sc[0][0] = x0.x; Sc[1][0] = x0.y; Sc[2][0] = x0.z; Sc[3][0] = x0.w;
    Sc[0][1] = x1.x; Sc[1][1] = x1.y; Sc[2][1] = x1.z; Sc[3][1] = x1.w;
  };
  int until_reload = 0;   // steps until the next checkpoint reload (unaligned C)
  int64_t reload_chunk = nchunks - 1;

  // The two roles of one timestep (kernel.rs:177-297). The row role needs
  // dsa of its own two rows only, which it sums itself, so it runs a batch of
  // kHalf steps ahead of the column role: it publishes dsa of every step of
  // the batch in dsab[buf], one barrier follows, and the column role reads
  // them. Partial sums go to part[] as [own block | other block], six per
  // step each (the row role's dv to dvp[] first).
  auto row_step = [&](int s, int buf, float* dvp) {
    // dS row += dy r^T (kernel.rs:248); dv, dsa (kernel.rs:261-262)
    float rr[4], kk[4], bb[4], ww[4], aa[4];
    unpack4(rr, tile(V_R, s)[L]);
    unpack4(kk, tile(V_K, s)[L]);
    unpack4(bb, tile(V_B, s)[L]);
    unpack4(ww, tile(V_W, s)[L]);
    unpack4(aa, tile(V_A, s)[L]);
    const float2 dyr = dyrow[s * 32];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      dSo[c] = __builtin_fmaf(dyr.x, rr[c], dSo[c]);
      dSt[c] = __builtin_fmaf(dyr.y, rr[c], dSt[c]);
    }
    // partial sums start from their first product (a product, not an FMA
    // with +0, which the compiler must keep as a three-operand VOP3 FMA)
    float dvo = dSo[0] * kk[0], dvt = dSt[0] * kk[0];
    float dsa_o = dSo[0] * bb[0], dsa_t = dSt[0] * bb[0];
#pragma unroll
    for (int c = 1; c < 4; ++c) {
      dvo = __builtin_fmaf(dSo[c], kk[c], dvo);
      dvt = __builtin_fmaf(dSt[c], kk[c], dvt);
      dsa_o = __builtin_fmaf(dSo[c], bb[c], dsa_o);
      dsa_t = __builtin_fmaf(dSt[c], bb[c], dsa_t);
    }
    row_pair_sum(dsa_o, dsa_t);
    // one lane per half-row publishes dsa of its own row; the others write a
    // sink, which keeps the step free of branches
    *((L & 7) == 0 ? &dsab[buf][s % kHalf][ro] : &dump[lane]) = dsa_o;
    // dS row = dS row * w~ + dsa a^T (kernel.rs:290-291)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      dSo[c] = __builtin_fmaf(dsa_o, aa[c], dSo[c] * ww[c]);
      dSt[c] = __builtin_fmaf(dsa_t, aa[c], dSt[c] * ww[c]);
    }
    dvp[2 * (s % kHalf)] = dvo;
    dvp[2 * (s % kHalf) + 1] = dvt;
  };
  auto col_step = [&](int s, int buf, float* part) {
    // dr from S_t; rebuild S_{t-1}; dS col += dy r; dw~, dk, db
    float dy[4], v[4], sa[4], ds[4];
    unpack4(dy, tile(V_DY, s)[L]);
    unpack4(v, tile(V_V, s)[L]);
    unpack4(sa, tile(V_SA, s)[L]);
    unpack4(ds, reinterpret_cast<const float4*>(dsab[buf][s % kHalf])[L]);   // dsa of rows 4L..
    const float4 prk = prec[(P_RK * kTile + s) * 32], pba = prec[(P_BA * kTile + s) * 32];
    const float4 pwi = prec[(P_WI * kTile + s) * 32];
    const float rc[2] = {prk.x, prk.y}, nkc[2] = {prk.z, prk.w};   // r, -k
    const float nbc[2] = {pba.x, pba.y}, ac[2] = {pba.z, pba.w};   // -b, a
    const float wc[2] = {pwi.x, pwi.y}, iwc[2] = {pwi.z, pwi.w};
    float drp[2], dwp[2], dkp[2], dbp[2], dap[2];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        // kernel.rs:230-237
        drp[d] = c == 0 ? Sc[c][d] * dy[c] : __builtin_fmaf(Sc[c][d], dy[c], drp[d]);
        // ((S - k v) - b sa) / w~, kernel.rs:239-246
        Sc[c][d] = __builtin_fmaf(nbc[d], sa[c], __builtin_fmaf(nkc[d], v[c], Sc[c][d])) * iwc[d];
        dSc[c][d] = __builtin_fmaf(rc[d], dy[c], dSc[c][d]);   // kernel.rs:249
        // kernel.rs:258-264
        dwp[d] = c == 0 ? dSc[c][d] * Sc[c][d] : __builtin_fmaf(dSc[c][d], Sc[c][d], dwp[d]);
        dkp[d] = c == 0 ? dSc[c][d] * v[c] : __builtin_fmaf(dSc[c][d], v[c], dkp[d]);
        dbp[d] = c == 0 ? dSc[c][d] * sa[c] : __builtin_fmaf(dSc[c][d], sa[c], dbp[d]);
        // da = S_{t-1}^T dsa (kernel.rs:280-287); dS col = dS col * w~ + a dsa (:293-294)
        dap[d] = c == 0 ? Sc[c][d] * ds[c] : __builtin_fmaf(Sc[c][d], ds[c], dap[d]);
        dSc[c][d] = __builtin_fmaf(ac[d], ds[c], dSc[c][d] * wc[d]);
      }
    float* po = part + O_COUNT * (s % kHalf);
    float* pt = part + O_COUNT * (kHalf + s % kHalf);
    po[O_DR] = drp[0];  pt[O_DR] = drp[1];
    po[O_DW] = dwp[0];  pt[O_DW] = dwp[1];
    po[O_DK] = dkp[0];  pt[O_DK] = dkp[1];
    po[O_DB] = dbp[0];  pt[O_DB] = dbp[1];
    po[O_DA] = dap[0];  pt[O_DA] = dap[1];
  };

  // Tile pipeline (tiles run backwards in time). While tile ti is computed,
  // the raw operands of tile ti-1 stream into LDS. At the tile end the
  // gradient partials are reduced and staged, one wait + barrier makes the
  // loads visible; the outputs of tile ti are flushed and tile ti-1 is
  // converted to fp32 (a different LDS region), a barrier, and the loads for
  // tile ti-2 are issued.
  const int ntiles = (T + kTile - 1) / kTile;
  auto tile_t0 = [&](int ti) { return ti * kTile; };
  auto tile_n = [&](int ti) { return min(kTile, T - ti * kTile); };
  if (ntiles > 0) {
    issue(tile_t0(ntiles - 1), tile_n(ntiles - 1), (ntiles - 1) & 1);
    __builtin_amdgcn_s_waitcnt(0);   // vmcnt/lgkmcnt 0
    lds_barrier();
    convert(tile_n(ntiles - 1));
    lds_barrier();
    if (ntiles > 1) issue(tile_t0(ntiles - 2), tile_n(ntiles - 2), (ntiles - 2) & 1);
  }

  // flush: threads 0..383, group fg = tid / 128 writes outputs 2fg and 2fg+1
  const int fg = tid >> 7;
  typedef Io<Tin> io;
  for (int ti = ntiles - 1; ti >= 0; --ti) {
    const int t0 = tile_t0(ti), nst = tile_n(ti);
    if constexpr (kCkTiled) {
      if (ck_needed(t0, nst)) {   // the reload of step t0 + kTile - 1
        const float4* ck = ckbuf[ti & 1];
        reload(ck[(ro * kHead + 4 * L) / 4], ck[(rt * kHead + 4 * L) / 4]);
      }
    }
    // the six gradients of own row/column 2q+up at step kHalf*hb + (L&7) of
    // a batch, from its reduce-scatter
    auto stage = [&](float* part, int hb) {
      const int so = kHalf * hb + (L & 7);
      // dw = W_SCALE * dw~ * w~ * sig * (1 - sig), kernel.rs:267-271
      part[O_DW] *= reinterpret_cast<const float*>(tile(V_DWF, so))[ro];
#pragma unroll
      for (int m = 0; m < O_COUNT; ++m) Io<Tin>::put1(&ost[m][so][ro], part[m]);
    };
    // step guard of the unaligned path: a partial first tile, and the
    // checkpoint reload at (t + 1) % C == 0 (kernel.rs:210-228)
    auto live = [&](int s) { return kCkTiled || s < nst; };
    auto col_reload = [&]() {
      if constexpr (!kCkTiled) {
        if (until_reload == 0) {
          until_reload = C;
          const float* src = ckpt_bh + reload_chunk * (kHead * kHead) + 4 * L;
          reload(*reinterpret_cast<const float4*>(src + ro * kHead),
                 *reinterpret_cast<const float4*>(src + rt * kHead));
          --reload_chunk;
        }
        --until_reload;
      }
    };
    constexpr int kBatches = kTile / kHalf;
    // Batches run later first. The row role of batch hb runs alone for the
    // last batch of the tile, and otherwise together with the column role of
    // batch hb+1 (no dependency between them); one barrier per batch.
    float dvb[kBatches][2 * kHalf];
#pragma unroll
    for (int s = kTile - 1; s >= kTile - kHalf; --s)
      if (live(s)) row_step(s, (kBatches - 1) & 1, dvb[kBatches - 1]);
#pragma unroll
    for (int hb = kBatches - 1; hb >= 0; --hb) {
      lds_barrier();   // dsa of batch hb visible
      float part[kParts];
#pragma unroll
      for (int k = kHalf - 1; k >= 0; --k) {
        const int s = kHalf * hb + k;
        if (live(s)) {
          col_reload();
          col_step(s, hb & 1, part);
        } else {
#pragma unroll
          for (int m = 0; m < O_COUNT; ++m) part[O_COUNT * k + m] = part[O_COUNT * (kHalf + k) + m] = 0.0f;
        }
        if (hb > 0 && live(s - kHalf)) row_step(s - kHalf, (hb - 1) & 1, dvb[hb - 1]);
      }
#pragma unroll
      for (int k = 0; k < kHalf; ++k) {
        part[O_COUNT * k + O_DV] = live(kHalf * hb + k) ? dvb[hb][2 * k] : 0.0f;
        part[O_COUNT * (kHalf + k) + O_DV] = live(kHalf * hb + k) ? dvb[hb][2 * k + 1] : 0.0f;
      }
      row16_reduce_scatter<kParts>(part, L);
      stage(part, hb);
    }

    // The loads of tile ti-1 have landed once vmcnt reaches 0 (they and the
    // stores of the previous tile end were issued a whole tile ago). Only LDS
    // is fenced by the barriers, so the stores below are not waited for until
    // the next tile end.
    __builtin_amdgcn_s_waitcnt(0);
    lds_barrier();
#pragma unroll
    for (int u = 0; u < kTile / 8; ++u) {
      const int st = sl + 8 * u;
      if (fg < 3 && st < nst) {
        const int64_t off = tok0 + (int64_t)(t0 + st) * tstride + 4 * pp;
        Tin* d0 = fg == 0 ? p.dv : fg == 1 ? p.dw : p.db;
        Tin* d1 = fg == 0 ? p.dr : fg == 1 ? p.dk : p.da;
        io::copy4(d0 + off, &ost[2 * fg][st][4 * pp]);
        io::copy4(d1 + off, &ost[2 * fg + 1][st][4 * pp]);
      }
    }
    if (ti > 0) convert(tile_n(ti - 1));
    lds_barrier();   // converted tile visible; `raw` free for the next loads
    if (ti > 1) issue(tile_t0(ti - 2), tile_n(ti - 2), (ti - 2) & 1);
  }

  if (p.ds0) {   // kernel.rs:299-307
    float* base = p.ds0 + bh * (kHead * kHead) + 4 * L;
    *reinterpret_cast<float4*>(base + ro * kHead) = make_float4(dSo[0], dSo[1], dSo[2], dSo[3]);
    *reinterpret_cast<float4*>(base + rt * kHead) = make_float4(dSt[0], dSt[1], dSt[2], dSt[3]);
  }
}

template <typename Tin>
hipError_t launch_bwd_t(const BackwardDesc& d, hipStream_t stream) {
  BwdParams<Tin> p;
  p.in[R_W] = static_cast<const Tin*>(d.w);
  p.in[R_R] = static_cast<const Tin*>(d.r);
  p.in[R_K] = static_cast<const Tin*>(d.k);
  p.in[R_V] = static_cast<const Tin*>(d.v);
  p.in[R_A] = static_cast<const Tin*>(d.a);
  p.in[R_B] = static_cast<const Tin*>(d.b);
  p.in[R_DY] = static_cast<const Tin*>(d.dy);
  p.ckpt = d.ckpt;
  p.sa = d.sa;
  p.dsT = d.dsT;
  p.dw = static_cast<Tin*>(d.dw);
  p.dr = static_cast<Tin*>(d.dr);
  p.dk = static_cast<Tin*>(d.dk);
  p.dv = static_cast<Tin*>(d.dv);
  p.da = static_cast<Tin*>(d.da);
  p.db = static_cast<Tin*>(d.db);
  p.ds0 = d.ds0;
  p.T = d.T;
  p.H = d.H;
  p.C = d.C;
  const dim3 grid(d.H, d.B, 1), block(kThreads, 1, 1);
  if (d.C % tile_len<Tin>() == 0)
    hipLaunchKernelGGL((wkv7_bwd_kernel<Tin, true>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((wkv7_bwd_kernel<Tin, false>), grid, block, 0, stream, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_backward(const BackwardDesc& d, hipStream_t stream) {
  if (d.B == 0 || d.H == 0) return hipSuccess;
  if (!d.kc.step_only) {
    if (chunk_backward_supported(d)) return launch_backward_chunked(d, stream);
    if (chunk_f32_backward_supported(d) && chunk_f32_backward_preferred(d))
      return launch_backward_chunked_f32(d, stream);
  }
  return d.dtype == Dtype::BF16 ? launch_bwd_t<bf16_t>(d, stream) : launch_bwd_t<float>(d, stream);
}

}  // namespace wkv7
