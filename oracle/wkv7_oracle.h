/*
 * TEST INFRASTRUCTURE ONLY -- not part of the product.
 *
 * CPU restatement of the rwkv-rs WKV7 kernels, used as the parity checker by
 * tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg. The
 * product path (rwkv-rs_amd/csrc) never links or calls this library.
 *
 * Tensor layouts follow the reference exactly:
 *   per-token tensors  [B, T, H, N]  row-major, N fastest
 *                      (crates/rwkv-nn/src/kernels/wkv7_common/kernel.rs:51-55)
 *   state / s0 / s_T   [B, H, N(value j), N(key i)]          (kernel.rs:29-35)
 *   checkpoints        [B, H, T/C, N(key i), N(value j)]     (kernel.rs:90-101)
 *
 * Every function returns 0 on success and a negative value on bad arguments.
 */
#ifndef WKV7_ORACLE_H
#define WKV7_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp32, reference operation order. kernel.rs:6-114 (wkv7_forward_kernel).
 * s0 and s_T may be NULL (use_initial_state / return_final_state = 0). */
int wkv7o_forward_f32(int64_t B, int64_t T, int64_t H, int64_t N, int64_t C,
                      const float *w, const float *r, const float *k,
                      const float *v, const float *a, const float *b,
                      const float *s0, float *ckpt, float *sa, float *y,
                      float *s_T, int nthreads);

/* fp32, reference operation order, state rebuilt by dividing by the decay and
 * reloaded from the checkpoint every C steps. kernel.rs:116-308
 * (wkv7_backward_kernel). ds_T and ds0 may be NULL. */
int wkv7o_backward_f32(int64_t B, int64_t T, int64_t H, int64_t N, int64_t C,
                       const float *w, const float *r, const float *k,
                       const float *v, const float *a, const float *b,
                       const float *ckpt, const float *sa, const float *dy,
                       const float *ds_T, float *dw, float *dr, float *dk,
                       float *dv, float *da, float *db, float *ds0,
                       int nthreads);

/* fp64 forward of the same recurrence (Appendix-A math of the reference,
 * kernel.rs:51-103). s0 / s_T may be NULL. */
int wkv7o_forward_f64(int64_t B, int64_t T, int64_t H, int64_t N,
                      const double *w, const double *r, const double *k,
                      const double *v, const double *a, const double *b,
                      const double *s0, double *y, double *s_T);

/* fp64 back-propagation through time that keeps every intermediate state
 * (no reversal). Computes the gradient of L = <dy, y> + <ds_T, s_T>.
 * ds_T / ds0 may be NULL. */
int wkv7o_grad_f64(int64_t B, int64_t T, int64_t H, int64_t N,
                   const double *w, const double *r, const double *k,
                   const double *v, const double *a, const double *b,
                   const double *s0, const double *dy, const double *ds_T,
                   double *dw, double *dr, double *dk, double *dv, double *da,
                   double *db, double *ds0);

/* fp32 slot-mapped inference forward. crates/rwkv-nn/src/kernels/wkv7_infer/
 * kernel.rs:15-114. `state` is [full_batch, H, N, N] and is updated in place
 * for the slots named by batch_ids. mask ([Ba, T], NULL = all ones): a zero
 * entry gives y = 0 and leaves the state untouched. use_dither adds
 * wkv7o_dither(elapsed_t[slot] + valid_t) to the decay (kernel.rs:75-77). */
int wkv7o_infer_f32(int64_t Ba, int64_t T, int64_t H, int64_t N,
                    int64_t full_batch, const float *w, const float *r,
                    const float *k, const float *v, const float *a,
                    const float *b, const int32_t *batch_ids, float *state,
                    const float *mask, const uint32_t *elapsed_t,
                    int use_dither, float *y);

/* The reference's inference kernel with element type F = bf16
 * (wkv7_infer/kernel.rs:15-114 instantiated at bf16, dither on per
 * wkv7_infer/host.rs:157 when use_dither = 1). Every F-typed value is a bf16:
 * the state read from and written back to the bf16 state buffer
 * (kernel.rs:35-42, 110-113), the operands staged in F (kernel.rs:66-70), the
 * decay computed in fp32 (plus the dither) and rounded to F once
 * (kernel.rs:71-78), and each F product and sum of the removal-state sum, the
 * state update and the output sum rounded to bf16, round to nearest even, in
 * the kernel's evaluation order (kernel.rs:81-98). All arrays are float32
 * holding bf16 values; `state` ([full_batch, H, N, N]) is updated in place and
 * keeps holding bf16 values. mask ([Ba, T], NULL = all ones) and elapsed_t as
 * for wkv7o_infer_f32. */
int wkv7o_infer_bf16(int64_t Ba, int64_t T, int64_t H, int64_t N,
                     int64_t full_batch, const float *w, const float *r,
                     const float *k, const float *v, const float *a,
                     const float *b, const int32_t *batch_ids, float *state,
                     const float *mask, const uint32_t *elapsed_t,
                     int use_dither, float *y);

/* float32 -> nearest bf16 (ties to even), returned as float32. */
float wkv7o_round_bf16(float x);

/* deterministic_dither, wkv7_infer/kernel.rs:8-13. */
float wkv7o_dither(uint32_t seed);

#ifdef __cplusplus
}
#endif

#endif /* WKV7_ORACLE_H */
