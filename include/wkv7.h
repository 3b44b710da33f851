/*
 * wkv7.h -- C ABI of the MI355X (gfx950) WKV7 time-mix recurrence.
 *
 * Drop-in boundary for the WKV7 operator of rwkv-rs (crate rwkv-nn). Every
 * entry point replaces one method of the reference's Burn backend traits and
 * keeps its argument order and meaning:
 *
 *   reference (under /root/reference/crates/rwkv-nn/src/kernels/)   entry point
 *   wkv7_pretrain/mod.rs:19-27   Wkv7PretrainBackend::wkv7_pretrain_forward     wkv7_pretrain_forward
 *   wkv7_pretrain/mod.rs:29-40   Wkv7PretrainBackend::wkv7_pretrain_backward    wkv7_pretrain_backward
 *   wkv7_statepass/mod.rs:19-28  Wkv7StatePassBackend::wkv7_statepass_forward   wkv7_statepass_forward
 *   wkv7_statepass/mod.rs:30-42  Wkv7StatePassBackend::wkv7_statepass_backward  wkv7_statepass_backward
 *   wkv7_statetune/mod.rs:19-28  Wkv7StateTuneBackend::wkv7_statetune_forward   wkv7_statetune_forward
 *   wkv7_statetune/mod.rs:30-41  Wkv7StateTuneBackend::wkv7_statetune_backward  wkv7_statetune_backward
 *   wkv7_infer/mod.rs:30-51      Wkv7InferBackend::wkv7_infer_forward           wkv7_infer_forward
 *   wkv7_common/host.rs:29-41    wkv7_forward_impl (flags)                      wkv7_forward
 *   wkv7_common/host.rs:185-199  wkv7_backward_impl (flags)                     wkv7_backward
 *
 * Operand names follow the reference: weight_decay (w, a raw logit; the
 * kernel forms exp(-e^{-1/2} sigmoid(w))), receptance (r), key (k), value
 * (v), removal (a), replacement (b). Layouts (row-major, last index fastest):
 *
 *   per-token tensors            [batch, context_len, num_heads, head_size]
 *   initial/final state, grads   [batch, num_heads, head_size(value), head_size(key)]   fp32
 *   state (checkpoints)          [batch, num_heads, context_len/chunk_len,
 *                                 head_size(key), head_size(value)]  fp32, i.e. the
 *                                state after step c*chunk_len + chunk_len - 1, transposed
 *   removal_state                [batch, context_len, num_heads, head_size]  fp32
 *
 * dtype (WKV7_DTYPE_*) is the element type of the per-token tensors and of
 * output / the six input gradients. State-family tensors (initial and final
 * state, checkpoints, removal_state, their gradients) are always fp32.
 *
 * Arithmetic. The reference casts non-fp32 inputs to fp32, computes in fp32
 * and casts the outputs back (wkv7_common/host.rs:45-64, 204-229). Here the
 * arithmetic depends on the kernel family a call runs on (WKV7_KERNELS_AUTO):
 *   - bf16 operands, forward at chunk_len 16, backward at chunk_len a multiple
 *     of 16 (the chunked matrix-core kernels): state, checkpoints,
 *     removal_state and every sum are fp32, but each product of two fp32
 *     quantities is formed from their bf16 halves as hi*hi + hi*lo + lo*hi,
 *     about 16 significant bits where fp32 has 24. Measured against the
 *     reference-order fp32 result: the state family about 3e-6 relative L2,
 *     the bf16 outputs and gradients at their own bf16 rounding (1e-4 to 7e-4);
 *   - the fp32 chunked kernels: the forward of fp32 operands at chunk_len
 *     16 and 32 and of bf16 operands at 32 (bf16 rows are widened to fp32
 *     exactly, as the reference casts them, and y is rounded to bf16 as it
 *     is stored), the backward of fp32 operands at chunk_len 16 and 32 and,
 *     past 32, with B*H >= 256 (where it is the faster family): fp32
 *     products on the fp32 matrix cores and fp32 sums, in the chunked matrix
 *     form (16-step blocks as matrix products rather than step by step); the
 *     backward rebuilds start states between checkpoints by the reference's
 *     reversal in its operation order, which amplifies any fp32 difference
 *     by about 1.35 per step. Measured against the reference-order fp32
 *     result at config[0]: output 2.6e-7 relative L2, checkpoints 1.7e-7,
 *     the gradients through the rebuilt start states (dw, dr, da) 6.2e-6,
 *     4.6e-6, 6.0e-6, the others 2.5e-7 to 4e-7 (the step kernels on the
 *     same call: 1.8e-7, 7e-8, 3.7e-6, 3.0e-6, 4.3e-6);
 *   - everything else (chunk lengths that are not multiples of 16, the
 *     forward past chunk_len 32, whose checkpoints in the reference's order
 *     keep the rebuilt-state gradients at the reference algorithm's own
 *     accuracy, and the fp32 backward past 32 with B*H < 256): the step
 *     kernels, fp32 products and sums in the reference's operation order.
 * wkv7_forward_ex / wkv7_backward_ex with WKV7_KERNELS_STEP run the step
 * kernels, i.e. the reference's operation order, for every case.
 *
 * Ownership and threading: the caller allocates every buffer on the device
 * (use wkv7_checkpoint_numel for the checkpoint tensor); the library
 * allocates nothing, keeps no state and is reentrant. Work is enqueued on
 * `stream` (a hipStream_t, NULL = the default stream) and the call returns
 * without synchronising. Outputs must not overlap each other or any input
 * (the infer state buffer, which is updated in place, is the only in/out
 * operand). Per-token tensors must be 8-byte aligned (bf16) or 16-byte
 * aligned (fp32); fp32 state-family tensors 16-byte aligned.
 *
 * Errors: every entry point returns WKV7_OK (0) or a wkv7_status code and never
 * aborts. All checks are done on the host before any HIP call; a failed
 * kernel launch returns WKV7_ERR_HIP and wkv7_last_hip_error() gives the
 * hipError_t of that failure on the calling thread. The reference panics on
 * the same conditions ("chunk_len must divide sequence length",
 * wkv7_common/host.rs:109-112).
 *
 * Supported shapes: head_size == 64 (RWKV-7's head size); batch_size and
 * num_heads up to 65535; context_len up to 2^31-1; context_len == 0 is
 * allowed (the final state is the initial state, the initial-state gradient
 * is the final-state gradient).
 *
 * Numerics: the backward rebuilds S_{t-1} = (S_t - v k^T - sa b^T) / w~ from
 * the last checkpoint, exactly like the reference (kernel.rs:239-246). Each
 * rebuilt step multiplies the rounding error by 1/w~ >= 1, so the gradient
 * error grows with chunk_len: about 4e-6 relative at chunk_len = 16, unusable
 * beyond about 32. The reference uses chunk_len = 16 (time_mixer/mod.rs:190).
 */
#ifndef RWKV_RS_AMD_WKV7_H
#define RWKV_RS_AMD_WKV7_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WKV7_ABI_VERSION 2

typedef enum wkv7_status {
  WKV7_OK = 0,
  WKV7_ERR_NULL_POINTER = 1, /* a required pointer is NULL */
  WKV7_ERR_SHAPE = 2,        /* negative or out-of-range dimension */
  WKV7_ERR_CHUNK_LEN = 3,    /* chunk_len <= 0 or does not divide context_len */
  WKV7_ERR_HEAD_SIZE = 4,    /* head_size != 64 */
  WKV7_ERR_DTYPE = 5,        /* unknown dtype code */
  WKV7_ERR_ALIGNMENT = 6,    /* a tensor pointer is misaligned */
  WKV7_ERR_OVERLAP = 7,      /* an output overlaps another operand */
  WKV7_ERR_FLAGS = 8,        /* a flag is not 0/1, contradicts a pointer, or
                                asks for the dither with an fp32 state */
  WKV7_ERR_HIP = 9,          /* the kernel launch failed */
  WKV7_ERR_SCRATCH_LIMIT = 10, /* the call needs more than the library's fixed
                                 scratch array (the _noalloc entry points) */
  WKV7_ERR_HANDOVER = 11      /* a chunked-forward launch gave up an internal
                                 wait; its outputs were poisoned with NaN
                                 (reported by wkv7_take_faults) */
} wkv7_status;

typedef enum wkv7_dtype { WKV7_DTYPE_F32 = 0, WKV7_DTYPE_BF16 = 1 } wkv7_dtype;

/* Library facts and error reporting. */
int wkv7_abi_version(void);
const char *wkv7_strerror(int status);
int wkv7_last_hip_error(void);

/* Number of fp32 elements of the checkpoint ("state") tensor,
 * batch * num_heads * (context_len / chunk_len) * head_size^2, or -1 when the
 * arguments are invalid. */
int64_t wkv7_checkpoint_numel(int64_t batch_size, int64_t context_len,
                              int64_t num_heads, int64_t head_size,
                              int64_t chunk_len);

/* ---------------------------------------------------------------------------
 * Generic forward: wkv7_forward_impl (wkv7_common/host.rs:29-183) with its two
 * flags. use_initial_state = 0 starts from zeros (initial_state may be NULL);
 * return_final_state = 0 skips final_state (may be NULL).
 * Outputs: state (checkpoints), removal_state, output, final_state.
 * ------------------------------------------------------------------------- */
int wkv7_forward(const void *weight_decay, const void *receptance,
                 const void *key, const void *value, const void *removal,
                 const void *replacement, const float *initial_state,
                 int64_t batch_size, int64_t context_len, int64_t num_heads,
                 int64_t head_size, int64_t chunk_len, int dtype,
                 int use_initial_state, int return_final_state, float *state,
                 float *removal_state, void *output, float *final_state,
                 void *stream);

/* ---------------------------------------------------------------------------
 * Generic backward: wkv7_backward_impl (wkv7_common/host.rs:185-369) with its
 * two flags. use_final_state_grad = 0 starts from a zero state gradient
 * (final_state_grad may be NULL); write_initial_state_grad = 0 skips
 * initial_state_grad (may be NULL).
 * ------------------------------------------------------------------------- */
int wkv7_backward(const void *weight_decay, const void *receptance,
                  const void *key, const void *value, const void *removal,
                  const void *replacement, const float *state,
                  const float *removal_state, const void *output_grad,
                  const float *final_state_grad, int64_t batch_size,
                  int64_t context_len, int64_t num_heads, int64_t head_size,
                  int64_t chunk_len, int dtype, int use_final_state_grad,
                  int write_initial_state_grad, void *weight_decay_grad,
                  void *receptance_grad, void *key_grad, void *value_grad,
                  void *removal_grad, void *replacement_grad,
                  float *initial_state_grad, void *stream);

/* ---------------------------------------------------------------------------
 * Explicit kernel choice. No counterpart in the reference (whose backend picks
 * one kernel per element type). wkv7_forward / wkv7_backward and the trait
 * entry points use WKV7_KERNELS_AUTO: the chunked matrix-core kernels for
 * bf16 operands (the forward at chunk_len 16 split-bf16 and at 32 on the
 * fp32 matrix cores, the backward at any multiple of 16) and for fp32
 * operands (the forward at chunk_len 16 and 32, the backward at 16 and 32
 * and, past 32, with B*H >= 256), the step-by-step kernels otherwise;
 * the arithmetic of each family is described at the top
 * of this file. WKV7_KERNELS_STEP runs the step kernels for every case (to
 * compare the families on one input). handover_spin_limit bounds the polls
 * of each hand-over wait inside the chunked forwards (0 = the default,
 * about 0.1 s); it exists so that tests can force the fault path below.
 * options may be NULL (all defaults).
 * ------------------------------------------------------------------------- */
typedef enum wkv7_kernels { WKV7_KERNELS_AUTO = 0, WKV7_KERNELS_STEP = 1 } wkv7_kernels;

typedef struct wkv7_options {
  int kernels;                  /* wkv7_kernels */
  uint32_t handover_spin_limit; /* 0 = default */
} wkv7_options;

int wkv7_forward_ex(const void *weight_decay, const void *receptance,
                    const void *key, const void *value, const void *removal,
                    const void *replacement, const float *initial_state,
                    int64_t batch_size, int64_t context_len, int64_t num_heads,
                    int64_t head_size, int64_t chunk_len, int dtype,
                    int use_initial_state, int return_final_state, float *state,
                    float *removal_state, void *output, float *final_state,
                    const wkv7_options *options, void *stream);

int wkv7_backward_ex(const void *weight_decay, const void *receptance,
                     const void *key, const void *value, const void *removal,
                     const void *replacement, const float *state,
                     const float *removal_state, const void *output_grad,
                     const float *final_state_grad, int64_t batch_size,
                     int64_t context_len, int64_t num_heads, int64_t head_size,
                     int64_t chunk_len, int dtype, int use_final_state_grad,
                     int write_initial_state_grad, void *weight_decay_grad,
                     void *receptance_grad, void *key_grad, void *value_grad,
                     void *removal_grad, void *replacement_grad,
                     float *initial_state_grad, const wkv7_options *options,
                     void *stream);

/* Hand-over faults of the chunked forwards (bf16 and fp32 operands). Their
 * producer and consumer waves pass chunks through LDS flags with bounded
 * waits. A wait that gives up
 * (which a correct kernel never does) makes the launch overwrite every output
 * of that (batch, head) -- output, removal_state, the checkpoints, the final
 * state -- with NaN, and adds one to a counter on the device. No counterpart
 * in the reference. wkv7_take_faults waits for `stream`, stores in *count the
 * number of such events on the current device since the previous call,
 * resets the counter, and returns WKV7_ERR_HANDOVER if *count > 0 (WKV7_OK
 * otherwise). Calls on one device must not overlap. */
int wkv7_take_faults(void *stream, uint32_t *count);

/* Device self-test of two bf16 building blocks, run exactly as the kernels
 * run them. No counterpart in the reference; it exists so that a toolchain
 * change that alters their lowering fails a test instead of shifting results
 * silently. For i < n, from the fp32 pairs (a[i], b[i]):
 *   split[2i], split[2i+1]: the packed bf16 hi parts (RNE(a), RNE(b); a in
 *     the low half) and lo parts (RNE(a - hi), RNE(b - hi)) with which the
 *     chunked kernels form their products of two fp32 quantities;
 *   sum[i]: RNE(a) + RNE(b) as an fp32 value, the sum the bf16-state decode
 *     rounds to bf16 (its bf16 rounding is that of the fp32 addition; the
 *     fp32 value can be one ulp off when one addend is below 2^-16 of the
 *     other).
 * Subnormal results are kept. Enqueued on `stream`; device pointers,
 * 4-byte aligned. */
int wkv7_selftest_bf16_ops(const float *a, const float *b, int64_t n,
                           uint32_t *split, float *sum, void *stream);

/* Wkv7PretrainBackend (wkv7_pretrain/mod.rs:18-41; CubeBackend impl
 * wkv7_pretrain/forward.rs:13-85): no initial state, no final state. */
int wkv7_pretrain_forward(const void *weight_decay, const void *receptance,
                          const void *key, const void *value,
                          const void *removal, const void *replacement,
                          int64_t batch_size, int64_t context_len,
                          int64_t num_heads, int64_t head_size,
                          int64_t chunk_len, int dtype, float *state,
                          float *removal_state, void *output, void *stream);

int wkv7_pretrain_backward(const void *weight_decay, const void *receptance,
                           const void *key, const void *value,
                           const void *removal, const void *replacement,
                           const float *state, const float *removal_state,
                           const void *output_grad, int64_t batch_size,
                           int64_t context_len, int64_t num_heads,
                           int64_t head_size, int64_t chunk_len, int dtype,
                           void *weight_decay_grad, void *receptance_grad,
                           void *key_grad, void *value_grad,
                           void *removal_grad, void *replacement_grad,
                           void *stream);

/* Wkv7StatePassBackend (wkv7_statepass/mod.rs:18-43; CubeBackend impl
 * wkv7_statepass/forward.rs:11-70): initial state in, final state out,
 * final-state gradient in, initial-state gradient out. */
int wkv7_statepass_forward(const void *weight_decay, const void *receptance,
                           const void *key, const void *value,
                           const void *removal, const void *replacement,
                           const float *initial_state, int64_t batch_size,
                           int64_t context_len, int64_t num_heads,
                           int64_t head_size, int64_t chunk_len, int dtype,
                           float *state, float *removal_state, void *output,
                           float *final_state, void *stream);

int wkv7_statepass_backward(const void *weight_decay, const void *receptance,
                            const void *key, const void *value,
                            const void *removal, const void *replacement,
                            const float *state, const float *removal_state,
                            const void *output_grad,
                            const float *final_state_grad, int64_t batch_size,
                            int64_t context_len, int64_t num_heads,
                            int64_t head_size, int64_t chunk_len, int dtype,
                            void *weight_decay_grad, void *receptance_grad,
                            void *key_grad, void *value_grad,
                            void *removal_grad, void *replacement_grad,
                            float *initial_state_grad, void *stream);

/* Wkv7StateTuneBackend (wkv7_statetune/mod.rs:18-42; CubeBackend impl
 * wkv7_statetune/forward.rs:19-76): initial state in, no final state,
 * initial-state gradient out. */
int wkv7_statetune_forward(const void *weight_decay, const void *receptance,
                           const void *key, const void *value,
                           const void *removal, const void *replacement,
                           const float *initial_state, int64_t batch_size,
                           int64_t context_len, int64_t num_heads,
                           int64_t head_size, int64_t chunk_len, int dtype,
                           float *state, float *removal_state, void *output,
                           void *stream);

int wkv7_statetune_backward(const void *weight_decay, const void *receptance,
                            const void *key, const void *value,
                            const void *removal, const void *replacement,
                            const float *state, const float *removal_state,
                            const void *output_grad, int64_t batch_size,
                            int64_t context_len, int64_t num_heads,
                            int64_t head_size, int64_t chunk_len, int dtype,
                            void *weight_decay_grad, void *receptance_grad,
                            void *key_grad, void *value_grad,
                            void *removal_grad, void *replacement_grad,
                            float *initial_state_grad, void *stream);

/* Wkv7InferBackend::wkv7_infer_forward (wkv7_infer/mod.rs:30-51; host
 * wkv7_infer/host.rs:27-187). Per-token tensors are
 * [active_batch_size, context_len, num_heads, 64] in dtype. Row b uses and
 * updates, in place, slot batch_ids[b] of `state` ([full_batch_size,
 * num_heads, 64, 64] in state_dtype); batch_ids must be distinct and in
 * [0, full_batch_size) (the reference asserts this in debug builds,
 * examples/rwkv-lm/src/inferring.rs:224-234; an out-of-range id gets output
 * 0 and touches no state). context_mask ([active_batch_size, context_len] in
 * dtype, NULL = all ones): a 0 entry gives output 0 and leaves the state
 * untouched.
 *
 * state_dtype selects which instantiation of the reference kernel runs:
 *   WKV7_DTYPE_F32   the reference at element type f32 (fp32 state and
 *                    arithmetic; bf16 operands are used as their exact fp32
 *                    values). No dither: use_dither must be 0, as the
 *                    reference's host sets it (host.rs:157).
 *   WKV7_DTYPE_BF16  the reference at element type bf16 (requires dtype
 *                    bf16): bf16 state, the decay rounded to bf16 after the
 *                    optional dither, and every product and sum of the update
 *                    and of the two sums over the key index rounded to bf16
 *                    (ties to even) in the kernel's order
 *                    (wkv7_infer/kernel.rs:71-98). The reference always
 *                    passes use_dither = 1 here (host.rs:157).
 * use_dither = 1 adds the reference's deterministic dither
 * (wkv7_infer/kernel.rs:8-13) seeded with elapsed_t[slot] + (unmasked steps
 * so far) to the fp32 decay before its rounding; elapsed_t
 * ([full_batch_size], read as uint32) may be NULL only when use_dither = 0.
 * The state buffer must be 16-byte aligned. */
int wkv7_infer_forward(const void *weight_decay, const void *receptance,
                       const void *key, const void *value, const void *removal,
                       const void *replacement, const int32_t *batch_ids,
                       void *state, const void *context_mask,
                       const int32_t *elapsed_t, int64_t active_batch_size,
                       int64_t context_len, int64_t num_heads,
                       int64_t head_size, int64_t full_batch_size, int dtype,
                       int state_dtype, int use_dither, void *output,
                       void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RWKV_RS_AMD_WKV7_H */
