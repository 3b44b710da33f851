/*
 * rwkv_lm_loss.h -- C ABI of the language model's training loss on gfx950:
 * the cross entropy of the next-token logits and l2wrap's gradient term,
 * fused into one forward and one backward pass over the logits.
 *
 *   reference (under /root/reference/)                                entry point
 *   examples/rwkv-lm/src/model.rs:158-169: l2wrap on the
 *     [batch * context_len, vocab] logits, then the mean
 *     CrossEntropyLoss over the rows                                  rwkv_cross_entropy_l2wrap_forward
 *   crates/rwkv-nn/src/kernels/l2wrap/mod.rs:38-66 (its backward
 *     adds 1e-4 / num_tokens * max(logits) at each row's argmax to
 *     the incoming gradient) with the cross entropy's backward       rwkv_cross_entropy_l2wrap_backward
 *
 * Forward, for each row r of logits ([rows, vocab] row-major in dtype) and
 * its target t_r (int64):
 *   lse_r  = log sum_j exp(x_rj)
 *   loss_r = lse_r - x_r,t_r
 * written to row_loss (fp32 [rows]; the loss is their mean), with row_lse,
 * row_max (fp32 [rows]) and row_argmax (int32 [rows]: the first index of
 * the row's maximum) kept for the backward. A target outside [0, vocab)
 * gives a NaN loss for its row and no target term in its gradient.
 *
 * Backward, with g_r = row_loss_grad[r] (fp32 [rows]; 1 / rows each when
 * the loss is the mean):
 *   dx_rj = g_r (exp(x_rj - lse_r) - [j == t_r]) + [j == argmax_r] l2wrap_scale max_r
 * written in dtype, where l2wrap_scale = 1e-4 / num_tokens
 * (l2wrap/mod.rs:61-62; 0 turns l2wrap off).
 *
 * Conventions are those of wkv7.h: wkv7_status return codes (checked on the
 * host before any launch), WKV7_DTYPE_* codes, work enqueued on `stream`
 * without synchronising, nothing allocated, outputs that must not overlap
 * any other operand. vocab is positive and below 2^31; when it is a
 * multiple of 8, logits and logits_grad are 16-byte aligned (rows are read
 * 8 logits at a time), otherwise aligned to their element; targets are
 * 8-byte aligned, the row arrays 4-byte.
 */
#ifndef RWKV_RS_AMD_LM_LOSS_H
#define RWKV_RS_AMD_LM_LOSS_H

#include <stddef.h>
#include <stdint.h>

#include "wkv7.h"

#ifdef __cplusplus
extern "C" {
#endif

int rwkv_cross_entropy_l2wrap_forward(const void *logits, const int64_t *targets,
                                      int64_t rows, int64_t vocab, int dtype,
                                      float *row_loss, float *row_lse, float *row_max,
                                      int32_t *row_argmax, void *stream);

int rwkv_cross_entropy_l2wrap_backward(const void *logits, const int64_t *targets,
                                       const float *row_lse, const float *row_max,
                                       const int32_t *row_argmax,
                                       const float *row_loss_grad, float l2wrap_scale,
                                       int64_t rows, int64_t vocab, int dtype,
                                       void *logits_grad, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RWKV_RS_AMD_LM_LOSS_H */
