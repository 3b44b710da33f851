// Matrix-core building blocks of the chunked WKV7 kernels (gfx950, bf16
// operands, fp32 accumulation).
//
// Chunked form. Within a chunk of L = 16 steps that starts from state S0,
// with the per-key log decays g_t = sum_{u<=t} log w~_u and gamma_t = e^{g_t}
// (gamma_0 = 1), the reference recurrence (wkv7_common/kernel.rs:63-102)
//   sa_t = S_{t-1} a_t,  S_t = S_{t-1} diag(w~_t) + sa_t b_t^T + v_t k_t^T,
//   y_t = S_t r_t
// unrolls into matrix products (rows of SA, Y, ... are the 16 steps):
//   A^ = a o gamma_{t-1},  R^ = r o gamma_t,  K~ = k / gamma_t,  B~ = b / gamma_t,
//   K- = k o gamma_L / gamma_t,  B- = b o gamma_L / gamma_t,
//   A_ab = strict_lower(A^ B~^T),  A_ak = strict_lower(A^ K~^T),
//   A_rb = lower(R^ B~^T),  A_rk = lower(R^ K~^T),  P = (I - A_ab)^{-1},
//   SA = P A^ S0^T + P A_ak V = W S0^T + U,
//   Y  = R^ S0^T + A_rk V + A_rb SA,
//   S_L = S0 diag(gamma_L) + V^T K- + SA^T B-.
// Only the last three lines depend on S0; everything else of a chunk is
// computed off the state's dependency chain.
//
// Accumulation chains. A chain of MFMAs that accumulate into the same
// registers uses one opcode throughout: on gfx950 a 16x16x16 result read as
// the accumulator of a following 16x16x32 (or the reverse) needs more wait
// states than the compiler inserts (measured: stale accumulator values with
// the two it emits), while same-opcode chains forward correctly back to
// back. 16x16x16 is used only for identity transposes, which start from zero
// and whose results are read by VALU instructions.
//
// Precision. Every product whose operands are both inexact in bf16 is formed
// from a hi/lo split (x = hi + lo, both bf16) as hi*hi + hi*lo + lo*hi with
// fp32 accumulation, which keeps about 16 significant bits per product.
// Products with a bf16 input tensor (v, or dy in the backward) as one operand
// split the other operand only.
//
// Fragment layouts (v_mfma_f32_16x16x16_bf16 and v_mfma_f32_16x16x32_bf16,
// lane l, quad qd = l / 16):
//   A operand  lane l holds A[row = l % 16][k = 4*qd + e]      (x16, e < 4)
//   B operand  lane l holds B[k = 4*qd + e][col = l % 16]       (x16)
//   result     lane l holds D[row = 4*qd + r][col = l % 16]     (r < 4)
// For x32 the operands hold 8 k-values per lane; the kernels use the k order
// k(e) = 16*(e / 4) + 4*qd + e % 4 within each 32-wide half of the key axis, so
// the two 4-value halves are exactly the result rows of two 16x16 tiles. With
// that order a state tile kept as a result (rows = key i, columns = value j)
// is directly the B operand of a contraction over i, and a result with rows =
// steps is directly the B operand of a contraction over steps; no transposes
// are needed on the state's chain.
#pragma once

#include "wkv7_device.hpp"

namespace wkv7 {
namespace chunk {

constexpr int kL = 16;          // steps per chunk
constexpr float kLog2e = 1.4426950408889634f;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct Split8 { bf16x8 hi, lo; };
struct Split4 { bf16x4 hi, lo; };

__device__ __forceinline__ f32x4 mma32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// hi*hi + hi*lo + lo*hi, small terms first
__device__ __forceinline__ f32x4 mma32x3(const Split8& a, const Split8& b, f32x4 c) {
  c = mma32(a.hi, b.lo, c);
  c = mma32(a.lo, b.hi, c);
  return mma32(a.hi, b.hi, c);
}
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// two values to bf16 hi and lo parts, one packed conversion each. The
// residual x - hi comes from one bf16 dot product per value, x + hi_pair .
// (-1, -0), instead of widening hi and subtracting (two instructions). x - hi
// is exact in fp32, so any rounding of the dot product gives it, and the
// split matches the subtraction bit for bit, subnormal residuals included,
// except where |x| rounds to infinity in bf16 (tests/test_gpu_selftest.py).
// The constants hold -0 rather than 0: this toolchain encodes (-1, 0) as the
// inline constant -1.0, which the instruction reads as another 16-bit value
// (measured: products of about hi / 128), while (-1, -0) stays a literal.
__device__ __forceinline__ void split2(float a, float b, uint32_t& hi, uint32_t& lo) {
  const bf16x2 h = __builtin_convertvector(f32x2{a, b}, bf16x2);
  const float la = __builtin_amdgcn_fdot2_f32_bf16(h, bf16x2{(__bf16)-1.0f, (__bf16)-0.0f}, a, false);
  const float lb = __builtin_amdgcn_fdot2_f32_bf16(h, bf16x2{(__bf16)-0.0f, (__bf16)-1.0f}, b, false);
  hi = __builtin_bit_cast(uint32_t, h);
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{la, lb}, bf16x2));
}
__device__ __forceinline__ Split4 split4(f32x4 x) {
  uint32_t h0, l0, h1, l1;
  split2(x[0], x[1], h0, l0);
  split2(x[2], x[3], h1, l1);
  return Split4{__builtin_bit_cast(bf16x4, make_uint2(h0, h1)),
                __builtin_bit_cast(bf16x4, make_uint2(l0, l1))};
}
// x32 fragment from two 4-value halves (the result rows of two tiles)
__device__ __forceinline__ bf16x8 cat8(bf16x4 a, bf16x4 b) {
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}
__device__ __forceinline__ Split8 split8(f32x4 x0, f32x4 x1) {
  const Split4 a = split4(x0), b = split4(x1);
  return Split8{cat8(a.hi, b.hi), cat8(a.lo, b.lo)};
}
__device__ __forceinline__ bf16x4 half_of(bf16x8 x, int h) {
  return h ? __builtin_shufflevector(x, x, 4, 5, 6, 7) : __builtin_shufflevector(x, x, 0, 1, 2, 3);
}
__device__ __forceinline__ Split4 half_of(const Split8& x, int h) {
  return Split4{half_of(x.hi, h), half_of(x.lo, h)};
}
__device__ __forceinline__ bf16x4 to_bf16x4(f32x4 x) {
  return __builtin_convertvector(x, bf16x4);
}

// Products over a 16-long axis on the 32-deep instruction: the k axis holds
// the hi part of the A operand in its first half and the lo part in its second
// (a "stacked" A operand); the B operand repeats the same 16 values in both
// halves. One instruction then forms a_hi b + a_lo b.
__device__ __forceinline__ bf16x8 stack(const Split4& a) { return cat8(a.hi, a.lo); }
__device__ __forceinline__ bf16x8 twice(bf16x4 b) { return cat8(b, b); }
// a (stacked, split) times b (exact in bf16), contraction length 16
__device__ __forceinline__ f32x4 mma_s2(bf16x8 a_stacked, bf16x4 b, f32x4 c) {
  return mma32(a_stacked, twice(b), c);
}
// a (stacked, split) times b (split), contraction length 16: three terms,
// a_hi b_lo from the B operand (b_lo | 0) and a_hi b_hi + a_lo b_hi
__device__ __forceinline__ f32x4 mma_s3(bf16x8 a_stacked, const Split4& b, f32x4 c) {
  c = mma32(a_stacked, cat8(b.lo, bf16x4{0, 0, 0, 0}), c);
  return mma32(a_stacked, twice(b.hi), c);
}

// X Y in the result layout from X^T and Y in the result layout (lane l holds
// M[4 qd + r][l % 16]): X^T's lanes are X as an A operand, Y's are Y as a B
// operand; split-bf16 product, contraction length 16. The operands come
// split (split4) so that a tile used several times is split once.
__device__ __forceinline__ f32x4 mma_tiles(const Split4& xt, const Split4& y, f32x4 c) {
  return mma_s3(stack(xt), y, c);
}
// P = (I - A)^-1 for a strictly triangular 16x16 A (lower or upper), from A
// and A^T in the result layout (t = l % 16, qd = l / 16); P in the result
// layout. Since A^16 = 0, P = (I + A)(I + A^2)(I + A^4)(I + A^8): eight
// products, five of them dependent, all operands in registers, each tile
// split into bf16 halves once.
__device__ __forceinline__ f32x4 unit_lower_inverse(f32x4 a, f32x4 at, int t, int qd) {
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  f32x4 id;
#pragma unroll
  for (int r = 0; r < 4; ++r) id[r] = (4 * qd + r == t) ? 1.0f : 0.0f;
  const Split4 sa = split4(a), sat = split4(at);
  const f32x4 a2 = mma_tiles(sat, sa, z), a2t = mma_tiles(sa, sat, z);
  const Split4 sa2 = split4(a2), sa2t = split4(a2t);
  const f32x4 a4 = mma_tiles(sa2t, sa2, z), a4t = mma_tiles(sa2, sa2t, z);
  const Split4 sa4t = split4(a4t);
  const f32x4 a8 = mma_tiles(sa4t, split4(a4), z);
  const f32x4 qt = mma_tiles(sa2, sat, id + at + a2t);   // ((I + A)(I + A^2))^T
  const f32x4 r = mma_tiles(sa4t, split4(a8), id + a4 + a8);    // (I + A^4)(I + A^8)
  return mma_tiles(split4(qt), split4(r), z);
}

// Transposed fragment load (ds_read_b64_tr_b16). Within each group of 16
// lanes, lane c supplies the address of 4 consecutive bf16 values; lane c' of
// the group receives value c' % 4 of the pieces addressed by lanes
// c' / 4 + 4 j, j = 0..3. If lane c of group g addresses row 4 g + c / 4,
// columns c0 + 4 (c % 4) of a row-major tile, lane l receives
// tile[4 qd + e][c0 + l % 16]: the x16 operand whose k index is the row.
__device__ __forceinline__ bf16x4 read_tr16(const void* lds) {
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  return __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4*)(__attribute__((address_space(3))) void*)(void*)lds));
}

// A tile of bf16 rows (64 columns) in LDS with each row's eight 16-byte
// pieces rotated: element (row, c) lives in piece (c / 8 + rot(row)) % 8,
// rot(row) = row + row / 8. The LDS (64 banks of 4 bytes) serves 32 lanes of
// an 8-byte read per cycle; with this rotation both 8-byte row reads of 16
// consecutive rows (the same piece of every row) and the transposed reads
// (32 bytes of 8 consecutive rows) hit every bank once (measured: no bank
// conflicts, where rot(row) = row gives two-way conflicts on the row reads).
__device__ __forceinline__ int tile_rot(int row) { return row + (row >> 3); }
// A row tile followed by 64 bytes: consecutive tiles (a value's hi and lo
// halves, or the rows of different inputs read by the same lanes) start 16
// banks apart. Unpadded, the two reads of a lane at the same place in two
// tiles hit one bank, and the compiler also pairs them into one read2/write2
// instruction, which serialises them (measured: two-way conflicts on every
// such pair).
struct PadTile {
  bf16_t r[kL][64];
  bf16_t pad[32];
};
static_assert(sizeof(PadTile) % 16 == 0, "16-byte aligned tiles");
__device__ __forceinline__ bf16_t* tile_at(bf16_t (*tile)[64], int row, int c) {
  return &tile[row][8 * (((c >> 3) + tile_rot(row)) & 7) + (c & 7)];
}
__device__ __forceinline__ const bf16_t* tile_at(const bf16_t (*tile)[64], int row, int c) {
  return &tile[row][8 * (((c >> 3) + tile_rot(row)) & 7) + (c & 7)];
}
__device__ __forceinline__ bf16x4 read4(const bf16_t (*tile)[64], int row, int c) {
  return *reinterpret_cast<const bf16x4*>(tile_at(tile, row, c));
}
__device__ __forceinline__ void write4(bf16_t (*tile)[64], int row, int c, bf16x4 v) {
  *reinterpret_cast<bf16x4*>(tile_at(tile, row, c)) = v;
}
// x32 fragment of one row (the lane's row), k over the 32 columns of half m
// in the kernels' k order: columns 32 m + 4 qd + e and 32 m + 16 + 4 qd + e
__device__ __forceinline__ bf16x8 row_frag(const bf16_t (*tile)[64], int row, int m, int qd) {
  return cat8(read4(tile, row, 32 * m + 4 * qd), read4(tile, row, 32 * m + 16 + 4 * qd));
}
// transposed x16 fragment of a rotated tile: lane l gets
// tile[row0 + 4 qd + e][c0 + l % 16] (k = row)
__device__ __forceinline__ bf16x4 tr_frag(const bf16_t (*tile)[64], int row0, int c0, int lane) {
  const int g = lane >> 4, c = lane & 15;
  return read_tr16(tile_at(tile, row0 + 4 * g + (c >> 2), c0 + 4 * (c & 3)));
}
// transposed x32 fragment, k = rows 32 m .. 32 m + 31 in the kernels' k order
__device__ __forceinline__ bf16x8 tr_frag32(const bf16_t (*tile)[64], int m, int c0, int lane) {
  return cat8(tr_frag(tile, 32 * m, c0, lane), tr_frag(tile, 32 * m + 16, c0, lane));
}

// inclusive prefix sum over the 16 lanes of a DPP row
__device__ __forceinline__ float row_scan16(float x) {
  x += dpp_mov<0x111>(x);   // row_shr:1
  x += dpp_mov<0x112>(x);   // row_shr:2
  x += dpp_mov<0x114>(x);   // row_shr:4
  x += dpp_mov<0x118>(x);   // row_shr:8
  return x;
}
// value of lane 15 of each DPP row, broadcast to the row
__device__ __forceinline__ float row_last16(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      0, __builtin_bit_cast(int, x), 0x15F, 0xf, 0xf, false));   // row_newbcast:15
}

// Sums over the four 16-lane rows of a wave (the quads qd of the MFMA
// layouts) without LDS, by gfx950's row-swapping moves (lane layout measured
// on the box): permlane16_swap(x, x) returns rows (0, 0, 2, 2) and (1, 1, 3,
// 3) of x, permlane32_swap(x, x) rows (0, 1, 0, 1) and (2, 3, 2, 3).
__device__ __forceinline__ float as_f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t as_u(float x) { return __float_as_uint(x); }
// x_0 + x_1 + x_2 + x_3 over the rows, in every lane
__device__ __forceinline__ float rows_total(float x) {
  const auto p = __builtin_amdgcn_permlane32_swap(as_u(x), as_u(x), false, false);
  const float s = as_f(p[0]) + as_f(p[1]);   // x_r + x_(r^2)
  const auto q = __builtin_amdgcn_permlane16_swap(as_u(s), as_u(s), false, false);
  return as_f(q[0]) + as_f(q[1]);
}
// sum of x over the rows below row qd (rows qd + 1 .. 3), in every lane of row qd
__device__ __forceinline__ float rows_after(float x, int qd) {
  const auto q = __builtin_amdgcn_permlane16_swap(as_u(x), as_u(x), false, false);
  const float pair = as_f(q[0]) + as_f(q[1]);   // x_0 + x_1 in rows 0, 1; x_2 + x_3 in rows 2, 3
  const auto p = __builtin_amdgcn_permlane32_swap(as_u(pair), as_u(pair), false, false);
  const float upper = as_f(p[1]);               // x_2 + x_3
  const float odd = as_f(q[1]);                 // x_1 in row 0, x_3 in row 2
  return qd == 0 ? odd + upper : qd == 1 ? upper : qd == 2 ? odd : 0.0f;
}

__device__ __forceinline__ float exp2_f(float x) { return __builtin_amdgcn_exp2f(x); }
// log2 of the decay: log2(w~) = W_SCALE * sigmoid(x) * log2(e)
__device__ __forceinline__ float log2_decay(float x) {
  const float sig = __builtin_amdgcn_rcpf(1.0f + exp2_f(-kLog2e * x));
  return (kWScale * kLog2e) * sig;
}

// this wave's LDS writes are done and visible to its own later reads
__device__ __forceinline__ void wave_lds_sync() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
  __builtin_amdgcn_wave_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Hand-over between the waves of a workgroup through LDS flags, for the
// chunked forwards whose preparing waves and chain waves run concurrently.
// polls of a hand-over flag before a wave gives up (each poll sleeps ~64
// cycles): about 0.1 s, far beyond any legitimate wait in a kernel that runs
// for well under a millisecond. The caller may lower it (tests force the
// fault path with a single poll).
constexpr uint32_t kSpinLimit = 1u << 22;

__device__ __forceinline__ int lds_load_flag(const int* f) {
  return __atomic_load_n(f, __ATOMIC_RELAXED);
}
__device__ __forceinline__ void lds_store_flag(int* f, int v) {
  __atomic_store_n(f, v, __ATOMIC_RELAXED);
}
// poll *f until it reaches v, at most `limit` times; false if it gave up
__device__ __forceinline__ bool wait_flag(const int* f, int v, uint32_t limit) {
  for (uint32_t n = 0; n < limit; ++n) {
    if (lds_load_flag(f) >= v) return true;
    __builtin_amdgcn_s_sleep(1);
  }
  return lds_load_flag(f) >= v;
}
// the wave's earlier LDS writes are complete before its later LDS accesses
__device__ __forceinline__ void lds_release() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
}
__device__ __forceinline__ void lds_acquire() {
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace chunk
}  // namespace wkv7
