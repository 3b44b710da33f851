/*
 * rwkv_neighbors.h -- C ABI of the ops on either side of the WKV7 operator in
 * an RWKV-7 time mixer, each side fused into one pass (gfx950).
 *
 *   reference (under /root/reference/crates/rwkv-nn/src/)             entry point
 *   kernels/token_shift_diff/mod.rs:28-36  TokenShiftDiffBackend::
 *     token_shift_diff (kernel.rs:17-64), then
 *   kernels/addcmul/mod.rs:24-40  AddcmulBackend::addcmul5 / addcmul
 *     (kernel.rs:4-53) on its difference, as
 *     modules/time_mixer/weight_prepare.rs:221-268 and
 *     modules/channel_mixer/mod.rs:96-106 call them                 rwkv_token_shift_mix_forward
 *   their autodiff backwards: token_shift_diff/backward.rs:34-101,
 *     addcmul/backward.rs:28-58                                      rwkv_token_shift_mix_backward
 *   modules/time_mixer/gated_readout.rs:126-145 (GroupNorm over
 *     heads, the r.k~.bonus term, the gate)                          rwkv_gated_readout_forward
 *   its autodiff backward (Burn's autodiff of the same ops)          rwkv_gated_readout_backward
 *   modules/time_mixer/weight_prepare.rs:282-317 (learning rate,
 *     replacement key, value residual, decay, normalized removal
 *     key, replacement), with the LoRA biases of
 *     layers/lora.rs:118-123                                          rwkv_weight_prepare_forward
 *   its autodiff backward (Burn's autodiff of the same ops)          rwkv_weight_prepare_backward
 *
 * Token shift + mixes. x ("embedded_context") is [batch, context_len, C]
 * row-major in dtype; for each row b and step t
 *   prev   = x[b, t-1] when t > 0 and step t-1 is valid, else the external
 *            shift embedded_token_shift[slot(b)] (zero when that is NULL)
 *   diff   = prev - x[b, t], or 0 when step t is masked
 *   mix_i  = x[b, t] + diff * scales[i, channel]          i < num_mixes
 * with slot(b) = batch_ids[b] (NULL: b). context_mask ([batch, context_len]
 * in dtype, NULL = all valid) holds 0/1. The mixes (and diff, if requested)
 * are written in out_dtype, which may differ from dtype (e.g. fp32 in,
 * bf16 out for the matrix products that consume them); diff stays fp32
 * between the shift and the mixes. next_token_shift ([full_batch_size, C]
 * in dtype, may be NULL) gets, at each active slot, x at the row's last
 * valid step, or the external shift when no step is valid; it may be the
 * embedded_token_shift buffer itself (the reference updates it in place).
 * The reference's WeightPrepare passes the five scales receptance,
 * weight_decay, key, value, learning_rate (num_mixes = 5); ChannelMixer one.
 * scales is [num_mixes, C] fp32, num_mixes in [0, 8].
 *
 * The backward takes the gradients of the mixes (num_mixes pointers, out
 * dtype, all required) and optionally of diff, and writes the gradient of x
 * (dtype), of the scales ([num_mixes, C] fp32) and, when
 * embedded_token_shift_grad is not NULL, of the external shift
 * ([full_batch_size, C] fp32; zero at slots no batch id names). The scale
 * gradients are reduced through a caller-provided workspace of
 * rwkv_token_shift_mix_workspace_bytes() bytes (16-byte aligned).
 *
 * Gated readout. For each row (batch, step) and head h, with y the WKV7
 * output and r, k~, v the operator's receptance, replacement key and value
 * ([rows, num_heads, 64] in dtype):
 *   out = (GroupNorm_h(y) * weight + bias + (sum_n r k~ bonus[h]) v) * gate
 * where GroupNorm_h normalises the head's 64 channels (biased variance,
 * epsilon) and gate, out are [rows, num_heads * 64] in act_dtype; bonus
 * ([num_heads, 64]), weight and bias ([num_heads * 64]) are fp32. The
 * backward writes the gradients of y, r, k~, v (dtype), gate (act_dtype) and
 * bonus, weight, bias (fp32, reduced through a workspace of
 * rwkv_gated_readout_workspace_bytes() bytes, 16-byte aligned); it recomputes
 * the row statistics from y.
 *
 * Conventions are those of wkv7.h: wkv7_status return codes (checked on the
 * host before any launch), WKV7_DTYPE_* codes, work enqueued on `stream`
 * without synchronising, nothing allocated, outputs that must not overlap
 * any other operand (except next_token_shift over embedded_token_shift).
 * Tensors must be 16-byte aligned (fp32) or 8-byte aligned (bf16), C (the
 * embedding width) a multiple of 4, head_size 64.
 */
#ifndef RWKV_RS_AMD_NEIGHBORS_H
#define RWKV_RS_AMD_NEIGHBORS_H

#include <stddef.h>
#include <stdint.h>

#include "wkv7.h"

#ifdef __cplusplus
extern "C" {
#endif

#define RWKV_MAX_MIXES 8

/* Workspace bytes for rwkv_token_shift_mix_backward, or -1 for invalid
 * arguments. */
int64_t rwkv_token_shift_mix_workspace_bytes(int64_t num_mixes, int64_t batch_size,
                                             int64_t context_len, int64_t embedded_dim);

int rwkv_token_shift_mix_forward(const void *embedded_context,
                                 const void *embedded_token_shift,
                                 const int32_t *batch_ids, const void *context_mask,
                                 const float *scales, int64_t num_mixes,
                                 int64_t batch_size, int64_t context_len,
                                 int64_t embedded_dim, int64_t full_batch_size,
                                 int dtype, int out_dtype, void *const *mixes,
                                 void *token_shifted_diff, void *next_token_shift,
                                 void *stream);

int rwkv_token_shift_mix_backward(const void *embedded_context,
                                  const void *embedded_token_shift,
                                  const int32_t *batch_ids, const void *context_mask,
                                  const float *scales, int64_t num_mixes,
                                  int64_t batch_size, int64_t context_len,
                                  int64_t embedded_dim, int64_t full_batch_size,
                                  int dtype, int out_dtype, const void *const *mix_grads,
                                  const void *token_shifted_diff_grad,
                                  void *embedded_context_grad,
                                  float *embedded_token_shift_grad, float *scales_grad,
                                  void *workspace, int64_t workspace_bytes, void *stream);

/* Workspace bytes for rwkv_gated_readout_backward, or -1 for invalid
 * arguments. */
int64_t rwkv_gated_readout_workspace_bytes(int64_t rows, int64_t num_heads,
                                           int64_t head_size);

int rwkv_gated_readout_forward(const void *wkv7_output, const void *receptance,
                               const void *replacement_key, const void *value,
                               const void *gate, const float *receptance_key_bonus,
                               const float *group_norm_weight,
                               const float *group_norm_bias, float epsilon,
                               int64_t rows, int64_t num_heads, int64_t head_size,
                               int dtype, int act_dtype, void *output, void *stream);

int rwkv_gated_readout_backward(const void *wkv7_output, const void *receptance,
                                const void *replacement_key, const void *value,
                                const void *gate, const float *receptance_key_bonus,
                                const float *group_norm_weight,
                                const float *group_norm_bias, float epsilon,
                                int64_t rows, int64_t num_heads, int64_t head_size,
                                int dtype, int act_dtype, const void *output_grad,
                                void *wkv7_output_grad, void *receptance_grad,
                                void *replacement_key_grad, void *value_grad,
                                void *gate_grad, float *receptance_key_bonus_grad,
                                float *group_norm_weight_grad,
                                float *group_norm_bias_grad, void *workspace,
                                int64_t workspace_bytes, void *stream);

/* Bytes of the device array that rwkv_gated_readout_backward_noalloc uses in
 * place of the workspace argument. */
#define RWKV_READOUT_SCRATCH_BYTES (4 * 1024 * 1024)

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving or training loops,
 * harnesses that forbid hipMalloc): rwkv_gated_readout_backward with the
 * workspace replaced by a fixed array of RWKV_READOUT_SCRATCH_BYTES that the
 * library holds on each GPU it runs on until the process ends. It allocates
 * nothing. Calls whose workspace (rwkv_gated_readout_workspace_bytes) would
 * exceed the array return WKV7_ERR_SCRATCH_LIMIT before any HIP call. Every
 * call on one GPU shares that GPU's array: calls that overlap in time on one
 * GPU (different streams without ordering between them) race and give wrong
 * parameter gradients; order them. The array's device address is looked up
 * on the first call per device, with that device current (that call may be
 * under graph capture), and kept for the life of the process: after a
 * hipDeviceReset of a device this entry point must not be called on it
 * again in the same process. Outputs equal rwkv_gated_readout_backward's
 * bit for bit. */
int rwkv_gated_readout_backward_noalloc(const void *wkv7_output, const void *receptance,
                                        const void *replacement_key, const void *value,
                                        const void *gate, const float *receptance_key_bonus,
                                        const float *group_norm_weight,
                                        const float *group_norm_bias, float epsilon,
                                        int64_t rows, int64_t num_heads, int64_t head_size,
                                        int dtype, int act_dtype, const void *output_grad,
                                        void *wkv7_output_grad, void *receptance_grad,
                                        void *replacement_key_grad, void *value_grad,
                                        void *gate_grad, float *receptance_key_bonus_grad,
                                        float *group_norm_weight_grad,
                                        float *group_norm_bias_grad, void *stream);

/*
 * End of the weight preparation. From the key and value projections
 * ("precursors") and the three LoRA products before their bias
 * (learning_rate_lora = act(x_a W_a) W_b, likewise weight_decay_lora and
 * value_residual_lora), all [rows, H * 64] in dtype, and the fp32 [H * 64]
 * parameters, per row and channel:
 *   lr                     = sigmoid(learning_rate_lora + learning_rate_bias)
 *   replacement_key        = key * (key_replacement * (lr - 1) + 1)
 *   value                  = lerp(value_precursor, value_from_first_cell,
 *                                 sigmoid(value_residual_lora + value_residual_bias))
 *   weight_decay           = -softplus(-(weight_decay_lora + weight_decay_bias)) - 0.5
 *   removal_key_normalized = -u,  u = rk / max(|rk|, 1e-12) over each head's 64
 *                            channels, rk = key * key_removal
 *   replacement            = u * lr
 * written in out_dtype (the WKV7 operand dtype). The value residual is on
 * when value_residual_bias is not NULL (every cell but the first); then
 * value_from_first_cell and value_residual_lora are required, otherwise they
 * must be NULL and value is the precursor. softplus(y) is y above 20.
 *
 * The backward takes the five outputs' gradients (out_dtype) and writes the
 * inputs' gradients (dtype; the residual's only when it is on) and the fp32
 * parameter gradients, summed over rows in a fixed order (workspace from
 * rwkv_weight_prepare_workspace_bytes). It recomputes the forward.
 */
int64_t rwkv_weight_prepare_workspace_bytes(int64_t rows, int64_t num_heads,
                                            int64_t head_size);

int rwkv_weight_prepare_forward(const void *key_precursor, const void *value_precursor,
                                const void *value_from_first_cell,
                                const void *learning_rate_lora, const void *weight_decay_lora,
                                const void *value_residual_lora,
                                const float *learning_rate_bias,
                                const float *weight_decay_bias,
                                const float *value_residual_bias,
                                const float *key_replacement, const float *key_removal,
                                int64_t rows, int64_t num_heads, int64_t head_size,
                                int dtype, int out_dtype, void *weight_decay,
                                void *replacement_key, void *value,
                                void *removal_key_normalized, void *replacement,
                                void *stream);

int rwkv_weight_prepare_backward(const void *key_precursor, const void *value_precursor,
                                 const void *value_from_first_cell,
                                 const void *learning_rate_lora,
                                 const void *weight_decay_lora,
                                 const void *value_residual_lora,
                                 const float *learning_rate_bias,
                                 const float *weight_decay_bias,
                                 const float *value_residual_bias,
                                 const float *key_replacement, const float *key_removal,
                                 int64_t rows, int64_t num_heads, int64_t head_size,
                                 int dtype, int out_dtype, const void *weight_decay_grad,
                                 const void *replacement_key_grad, const void *value_grad,
                                 const void *removal_key_normalized_grad,
                                 const void *replacement_grad, void *key_precursor_grad,
                                 void *value_precursor_grad,
                                 void *value_from_first_cell_grad,
                                 void *learning_rate_lora_grad,
                                 void *weight_decay_lora_grad,
                                 void *value_residual_lora_grad,
                                 float *learning_rate_bias_grad,
                                 float *weight_decay_bias_grad,
                                 float *value_residual_bias_grad,
                                 float *key_replacement_grad, float *key_removal_grad,
                                 void *workspace, int64_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RWKV_RS_AMD_NEIGHBORS_H */
