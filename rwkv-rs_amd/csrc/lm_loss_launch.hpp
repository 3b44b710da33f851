// Launchers of the fused cross entropy + l2wrap kernels (lm_loss.hip). The C
// ABI (lm_loss_api.cpp) checks every argument before it calls these.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace rwkv_loss {

constexpr int kThreads = 256;   // one block per row
constexpr int kPiece = 8;       // logits per 16-byte (bf16) or 32-byte (fp32) access

struct XentArgs {
  const void* logits;        // [rows, vocab]
  const int64_t* targets;    // [rows]
  int64_t rows, vocab;
  bool bf16;
  float *row_loss, *row_lse, *row_max;   // forward outputs
  int32_t* row_argmax;
  const float *lse, *max;                // backward inputs (the forward's outputs)
  const int32_t* argmax;
  const float* row_grad;
  float l2wrap_scale;
  void* logits_grad;         // backward output, [rows, vocab]
};

hipError_t launch_xent_forward(const XentArgs& a, hipStream_t s);
hipError_t launch_xent_backward(const XentArgs& a, hipStream_t s);

}  // namespace rwkv_loss
