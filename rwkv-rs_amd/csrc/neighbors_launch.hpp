// Launchers of the kernels that neighbour the WKV7 operator in a time mixer:
// the token shift with its channel mixes and the element-wise end of the
// weight preparation before it, and the gated readout (GroupNorm, bonus,
// gate) after it. The C ABI (neighbors_api.cpp) checks
// every argument before it calls these.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace rwkv_nb {

constexpr int kMaxMixes = 8;        // channel mixes of one token shift
constexpr int kMixRowsPerWave = 8;  // rows (batch, step) one wave walks
constexpr int kMixRowsPerBlock = 4 * kMixRowsPerWave;
constexpr int kMixColsPerBlock = 256;  // 64 lanes x 4 channels
constexpr int kReadoutRowsPerGroup = 4;  // rows one 16-lane group walks
constexpr int kReadoutRowsPerBlock = 16 * kReadoutRowsPerGroup;
constexpr int kReadoutSums = 3;     // group-norm weight, bias, bonus
constexpr int kPrepareRowsPerGroup = 4;  // rows one 16-lane group walks
constexpr int kPrepareRowsPerBlock = 16 * kPrepareRowsPerGroup;
// column sums of the weight-preparation backward, in workspace order: the
// learning-rate, decay and value-residual LoRA biases, key replacement and
// key removal (the value-residual slot only when the cell has one)
enum { PS_LR_BIAS, PS_WD_BIAS, PS_KEY_REPLACEMENT, PS_KEY_REMOVAL, PS_VR_BIAS, kPrepareSums };
static_assert(kPrepareSums <= kMaxMixes, "one column-sum launch serves at most kMaxMixes sums");

struct ShiftMixArgs {
  const void* x;             // [rows, C] (rows = batch * T), dtype x_bf16
  const void* shift;         // [full_batch, C] or null (zeros)
  const int32_t* batch_ids;  // [batch] or null (identity)
  const void* mask;          // [batch, T] in x's dtype, or null (all valid)
  const float* scales;       // [num_mixes, C]
  int64_t batch, T, C, full_batch;
  int num_mixes;
  bool x_bf16, out_bf16;
  void* mixes[kMaxMixes];    // forward: [rows, C] each, out dtype
  void* diff;                // forward: [rows, C] out dtype, or null
  void* next_shift;          // forward: [full_batch, C] x dtype, or null
  const void* mix_grads[kMaxMixes];  // backward: [rows, C] out dtype
  const void* diff_grad;     // backward: [rows, C] out dtype, or null
  void* x_grad;              // backward: [rows, C] x dtype
  float* shift_grad;         // backward: [full_batch, C] or null
  float* scales_grad;        // backward: [num_mixes, C]
  float* workspace;          // backward: [row_blocks, num_mixes, C]
};

struct ReadoutArgs {
  const void *y, *r, *k, *v;  // [rows, H, 64], operand dtype
  const void* gate;           // [rows, H * 64], activation dtype
  const float* bonus;         // [H, 64]
  const float* weight;        // [H * 64]
  const float* bias;          // [H * 64]
  float eps;
  int64_t rows, H;
  bool op_bf16, act_bf16;
  void* out;                  // forward: [rows, H * 64], activation dtype
  const void* out_grad;       // backward: [rows, H * 64], activation dtype
  void *y_grad, *r_grad, *k_grad, *v_grad;  // backward: operand dtype
  void* gate_grad;            // backward: activation dtype
  float *bonus_grad, *weight_grad, *bias_grad;  // backward
  float* workspace;           // backward: [row_blocks, 3, H * 64]
};

struct PrepareArgs {
  const void *key, *value;    // [rows, H * 64] precursors, input dtype
  const void* value_first;    // [rows, H * 64] or null (the first cell: no residual)
  const void *lr, *wd;        // LoRA products before their bias, input dtype
  const void* vr;             // the value-residual LoRA product; null iff value_first is
  const float *lr_bias, *wd_bias, *vr_bias;          // [H * 64]; vr_bias null iff vr is
  const float *key_replacement, *key_removal;        // [H * 64]
  int64_t rows, H;
  bool in_bf16, out_bf16;
  bool residual;              // the cell has a value residual (vr_bias set; every cell but the first)
  // forward outputs / backward output gradients, [rows, H * 64], out dtype
  void *weight_decay, *replacement_key, *value_out, *removal, *replacement;
  const void *weight_decay_grad, *replacement_key_grad, *value_out_grad, *removal_grad,
      *replacement_grad;
  // backward: input gradients (input dtype) and parameter gradients
  void *key_grad, *value_grad, *value_first_grad, *lr_grad, *wd_grad, *vr_grad;
  float* sums[kPrepareSums];  // [H * 64] each, in the order above
  float* workspace;           // [row_blocks, sums used, H * 64]
};

inline int64_t mix_row_blocks(int64_t rows) {
  return (rows + kMixRowsPerBlock - 1) / kMixRowsPerBlock;
}
inline int64_t readout_row_blocks(int64_t rows) {
  return (rows + kReadoutRowsPerBlock - 1) / kReadoutRowsPerBlock;
}
inline int64_t prepare_row_blocks(int64_t rows) {
  return (rows + kPrepareRowsPerBlock - 1) / kPrepareRowsPerBlock;
}

hipError_t launch_shift_mix_forward(const ShiftMixArgs& a, hipStream_t s);
hipError_t launch_shift_mix_backward(const ShiftMixArgs& a, hipStream_t s);
hipError_t launch_readout_forward(const ReadoutArgs& a, hipStream_t s);
hipError_t launch_readout_backward(const ReadoutArgs& a, hipStream_t s);
hipError_t launch_prepare_forward(const PrepareArgs& a, hipStream_t s);
hipError_t launch_prepare_backward(const PrepareArgs& a, hipStream_t s);

// Size of the library's fixed device array that stands in for the gated
// readout backward's workspace, and its device address on the current device
// (looked up on the first call per device; no allocation).
constexpr int64_t kReadoutScratchBytes = int64_t(4) << 20;
hipError_t readout_scratch(float** out);

}  // namespace rwkv_nb
