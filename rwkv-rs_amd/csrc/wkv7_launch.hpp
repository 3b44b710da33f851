// Internal launch interface between the C ABI (wkv7_api.cpp) and the kernels.
// Shapes are validated by the ABI layer before any of these is called.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wkv7 {

constexpr int kHeadSize = 64;   // the kernels are specialised for N = 64

enum class Dtype : int { F32 = 0, BF16 = 1 };

// kernel family (WKV7_KERNELS_*) and the chunked forward's hand-over bound
struct KernelChoice {
  bool step_only = false;       // WKV7_KERNELS_STEP
  uint32_t spin_limit = 0;      // 0 = default
};

// Forward pass, mirrors wkv7_forward_impl (wkv7_common/host.rs:29-183).
struct ForwardDesc {
  Dtype dtype;
  int B, T, H, C;               // batch, context length, heads, chunk_len
  const void *w, *r, *k, *v, *a, *b;   // [B,T,H,64] in dtype
  const float* s0;              // [B,H,64,64] or nullptr (zeros)
  float* ckpt;                  // [B,H,T/C,64,64], key-major (transposed)
  float* sa;                    // [B,T,H,64] removal_state
  void* y;                      // [B,T,H,64] in dtype
  float* sT;                    // [B,H,64,64] or nullptr
  KernelChoice kc;
};

// Backward pass, mirrors wkv7_backward_impl (wkv7_common/host.rs:185-369).
struct BackwardDesc {
  Dtype dtype;
  int B, T, H, C;
  const void *w, *r, *k, *v, *a, *b;   // [B,T,H,64] in dtype
  const float* ckpt;            // [B,H,T/C,64,64]
  const float* sa;              // [B,T,H,64]
  const void* dy;               // [B,T,H,64] in dtype
  const float* dsT;             // [B,H,64,64] or nullptr (zeros)
  void *dw, *dr, *dk, *dv, *da, *db;   // [B,T,H,64] in dtype
  float* ds0;                   // [B,H,64,64] or nullptr
  KernelChoice kc;
};

// Slot-mapped inference, mirrors wkv7_infer_forward_impl
// (wkv7_infer/host.rs:27-187).
struct InferDesc {
  Dtype dtype;
  Dtype state_dtype;            // fp32, or bf16 (then dtype is bf16 too)
  int Ba, T, H, full_batch;
  const void *w, *r, *k, *v, *a, *b;   // [Ba,T,H,64] in dtype
  const int32_t* batch_ids;     // [Ba], values in [0, full_batch)
  void* state;                  // [full_batch,H,64,64] in state_dtype, updated in place
  const void* context_mask;     // [Ba,T] in dtype, or nullptr (all ones)
  const int32_t* elapsed_t;     // [full_batch] (read as u32), or nullptr
  int use_dither;
  void* y;                      // [Ba,T,H,64] in dtype
};

hipError_t launch_forward(const ForwardDesc& d, hipStream_t stream);

// Chunked matrix-core forward (wkv7_chunk_forward.hip): bf16 operands,
// chunk_len 16. launch_forward picks it when supported, unless the caller
// asked for the step kernels (KernelChoice::step_only).
bool chunk_forward_supported(const ForwardDesc& d);
hipError_t launch_forward_chunked(const ForwardDesc& d, hipStream_t stream);
// the chunked forwards' hand-over fault counter on the current device: read
// and reset on `stream`, then wait for it
hipError_t take_handover_faults(hipStream_t stream, uint32_t* count);
// that counter's device address on the current device
hipError_t handover_fault_counter(unsigned int** counter);

// Chunked fp32 matrix-core forward (wkv7_f32_chunk.hip): fp32 operands at
// chunk_len 16 and 32, bf16 operands at 32; picked by launch_forward under
// the same choice. Its hand-over faults count in the same counter.
bool chunk_f32_forward_supported(const ForwardDesc& d);
hipError_t launch_forward_chunked_f32(const ForwardDesc& d, hipStream_t stream);

// Chunked matrix-core backward (wkv7_chunk_backward.hip): bf16 operands,
// chunk_len a multiple of 16, T a positive multiple of chunk_len; picked by
// launch_backward under the same choice.
bool chunk_backward_supported(const BackwardDesc& d);
hipError_t launch_backward_chunked(const BackwardDesc& d, hipStream_t stream);
// Chunked fp32 matrix-core backward (wkv7_f32_chunk.hip): fp32 operands,
// chunk_len a multiple of 16, T a positive multiple of chunk_len; picked by
// launch_backward where chunk_f32_backward_preferred holds as well, the step
// kernels otherwise.
bool chunk_f32_backward_supported(const BackwardDesc& d);
bool chunk_f32_backward_preferred(const BackwardDesc& d);
hipError_t launch_backward_chunked_f32(const BackwardDesc& d, hipStream_t stream);
hipError_t launch_backward(const BackwardDesc& d, hipStream_t stream);
hipError_t launch_infer(const InferDesc& d, hipStream_t stream);

// Device self-test of the bf16 split and rounded sum (wkv7_selftest.hip);
// n <= 2^31 * 256 pairs, pointers checked by the ABI layer.
hipError_t launch_bf16_ops_selftest(const float* a, const float* b, int64_t n, uint32_t* split,
                                    float* sum, hipStream_t stream);

// WKV7_OK for hipSuccess; otherwise records e for wkv7_last_hip_error() on
// the calling thread and returns WKV7_ERR_HIP
int hip_status(hipError_t e);

}  // namespace wkv7
