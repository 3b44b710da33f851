// C ABI of the WKV7 kernels: argument validation and dispatch.
//
// Every check happens here, on the host, before any HIP call, so that a bad
// call returns a status code instead of launching a kernel whose grid or
// indexing does not match its buffers. The reference panics on the same
// conditions (wkv7_common/host.rs:109-112 and the unwraps at :175, :358).
#include "../../include/wkv7.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <initializer_list>
#include <vector>

#include "wkv7_launch.hpp"

namespace {

thread_local int g_last_hip_error = 0;

constexpr int64_t kN = wkv7::kHeadSize;
constexpr int64_t kMaxGridDim = 65535;

struct Range {
  const void* p;
  int64_t bytes;
};

bool overlaps(const Range& x, const Range& y) {
  if (!x.p || !y.p || x.bytes <= 0 || y.bytes <= 0) return false;
  const auto a0 = reinterpret_cast<uintptr_t>(x.p), b0 = reinterpret_cast<uintptr_t>(y.p);
  return a0 < b0 + static_cast<uintptr_t>(y.bytes) && b0 < a0 + static_cast<uintptr_t>(x.bytes);
}

// outputs must not overlap each other or any input
bool any_overlap(const std::vector<Range>& outs, const std::vector<Range>& ins) {
  for (size_t i = 0; i < outs.size(); ++i) {
    for (size_t j = i + 1; j < outs.size(); ++j)
      if (overlaps(outs[i], outs[j])) return true;
    for (const Range& in : ins)
      if (overlaps(outs[i], in)) return true;
  }
  return false;
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

struct Shape {
  int64_t B, T, H, C;
  int64_t tok_elems() const { return B * T * H * kN; }
  int64_t state_elems() const { return B * H * kN * kN; }
  int64_t ckpt_elems() const { return B * H * (T / C) * kN * kN; }
};

int check_dtype(int dtype) {
  return (dtype == WKV7_DTYPE_F32 || dtype == WKV7_DTYPE_BF16) ? WKV7_OK : WKV7_ERR_DTYPE;
}

int elem_bytes(int dtype) { return dtype == WKV7_DTYPE_BF16 ? 2 : 4; }

// true when the product of the non-negative factors fits in int64
bool product_fits(std::initializer_list<int64_t> factors) {
  int64_t acc = 1;
  for (int64_t f : factors)
    if (__builtin_mul_overflow(acc, f, &acc)) return false;
  return true;
}

// shape checks shared by forward and backward; C is the chunk length. Every
// byte count the checks below form (per-token tensors, checkpoints) must fit
// in int64.
int check_shape(int64_t B, int64_t T, int64_t H, int64_t N, int64_t C, int dtype) {
  if (int rc = check_dtype(dtype)) return rc;
  if (N != kN) return WKV7_ERR_HEAD_SIZE;
  if (B < 0 || T < 0 || H < 0) return WKV7_ERR_SHAPE;
  if (B > kMaxGridDim || H > kMaxGridDim || T > INT32_MAX) return WKV7_ERR_SHAPE;
  if (C <= 0 || C > INT32_MAX || T % C != 0) return WKV7_ERR_CHUNK_LEN;
  if (!product_fits({B, T, H, kN, 4}) || !product_fits({B, H, T / C, kN * kN, 4}))
    return WKV7_ERR_SHAPE;
  return WKV7_OK;
}

int check_flag(int f) { return (f == 0 || f == 1) ? WKV7_OK : WKV7_ERR_FLAGS; }

int kernel_choice(const wkv7_options* o, wkv7::KernelChoice* kc) {
  *kc = wkv7::KernelChoice{};
  if (!o) return WKV7_OK;
  if (o->kernels != WKV7_KERNELS_AUTO && o->kernels != WKV7_KERNELS_STEP) return WKV7_ERR_FLAGS;
  kc->step_only = o->kernels == WKV7_KERNELS_STEP;
  kc->spin_limit = o->handover_spin_limit;
  return WKV7_OK;
}

}  // namespace

namespace wkv7 {
int hip_status(hipError_t e) {
  if (e == hipSuccess) return WKV7_OK;
  g_last_hip_error = static_cast<int>(e);
  return WKV7_ERR_HIP;
}
}  // namespace wkv7

using wkv7::hip_status;

extern "C" {

int wkv7_abi_version(void) { return WKV7_ABI_VERSION; }

int wkv7_selftest_bf16_ops(const float* a, const float* b, int64_t n, uint32_t* split,
                           float* sum, void* stream) {
  if (n < 0 || n > (int64_t)INT32_MAX * 256) return WKV7_ERR_SHAPE;
  if (n == 0) return WKV7_OK;
  if (!a || !b || !split || !sum) return WKV7_ERR_NULL_POINTER;
  if (!aligned(a, 4) || !aligned(b, 4) || !aligned(split, 4) || !aligned(sum, 4))
    return WKV7_ERR_ALIGNMENT;
  const std::vector<Range> ins = {{a, n * 4}, {b, n * 4}};
  const std::vector<Range> outs = {{split, n * 8}, {sum, n * 4}};
  if (any_overlap(outs, ins)) return WKV7_ERR_OVERLAP;
  return hip_status(
      wkv7::launch_bf16_ops_selftest(a, b, n, split, sum, static_cast<hipStream_t>(stream)));
}

int wkv7_last_hip_error(void) { return g_last_hip_error; }

int wkv7_take_faults(void* stream, uint32_t* count) {
  if (!count) return WKV7_ERR_NULL_POINTER;
  *count = 0;
  if (int rc = hip_status(wkv7::take_handover_faults(static_cast<hipStream_t>(stream), count)))
    return rc;
  return *count > 0 ? WKV7_ERR_HANDOVER : WKV7_OK;
}

const char* wkv7_strerror(int status) {
  switch (status) {
    case WKV7_OK: return "ok";
    case WKV7_ERR_NULL_POINTER: return "a required pointer is NULL";
    case WKV7_ERR_SHAPE: return "negative or out-of-range dimension";
    case WKV7_ERR_CHUNK_LEN: return "chunk_len must divide sequence length";
    case WKV7_ERR_HEAD_SIZE: return "head_size must be 64";
    case WKV7_ERR_DTYPE: return "unknown dtype (expected WKV7_DTYPE_F32 or WKV7_DTYPE_BF16)";
    case WKV7_ERR_ALIGNMENT: return "tensor pointer is misaligned";
    case WKV7_ERR_OVERLAP: return "an output buffer overlaps another operand";
    case WKV7_ERR_FLAGS:
      return "invalid flag value, flag/pointer mismatch, or dither asked for an fp32 state";
    case WKV7_ERR_HIP: return "HIP kernel launch failed";
    case WKV7_ERR_HANDOVER:
      return "a chunked forward gave up an internal hand-over wait; its outputs are NaN";
    case WKV7_ERR_SCRATCH_LIMIT:
      return "the call needs more scratch memory than the library's fixed device array holds";
    default: return "unknown wkv7 status";
  }
}

int64_t wkv7_checkpoint_numel(int64_t batch_size, int64_t context_len, int64_t num_heads,
                              int64_t head_size, int64_t chunk_len) {
  if (check_shape(batch_size, context_len, num_heads, head_size, chunk_len, WKV7_DTYPE_F32))
    return -1;
  return Shape{batch_size, context_len, num_heads, chunk_len}.ckpt_elems();
}

int wkv7_forward(const void* weight_decay, const void* receptance, const void* key,
                 const void* value, const void* removal, const void* replacement,
                 const float* initial_state, int64_t batch_size, int64_t context_len,
                 int64_t num_heads, int64_t head_size, int64_t chunk_len, int dtype,
                 int use_initial_state, int return_final_state, float* state,
                 float* removal_state, void* output, float* final_state, void* stream) {
  return wkv7_forward_ex(weight_decay, receptance, key, value, removal, replacement,
                         initial_state, batch_size, context_len, num_heads, head_size,
                         chunk_len, dtype, use_initial_state, return_final_state, state,
                         removal_state, output, final_state, nullptr, stream);
}

int wkv7_forward_ex(const void* weight_decay, const void* receptance, const void* key,
                    const void* value, const void* removal, const void* replacement,
                    const float* initial_state, int64_t batch_size, int64_t context_len,
                    int64_t num_heads, int64_t head_size, int64_t chunk_len, int dtype,
                    int use_initial_state, int return_final_state, float* state,
                    float* removal_state, void* output, float* final_state,
                    const wkv7_options* options, void* stream) {
  wkv7::KernelChoice kc;
  if (int rc = kernel_choice(options, &kc)) return rc;
  if (int rc = check_shape(batch_size, context_len, num_heads, head_size, chunk_len, dtype))
    return rc;
  if (int rc = check_flag(use_initial_state)) return rc;
  if (int rc = check_flag(return_final_state)) return rc;
  const Shape sh{batch_size, context_len, num_heads, chunk_len};
  const int64_t tok = sh.tok_elems() * elem_bytes(dtype);
  const int64_t st = sh.state_elems() * 4;
  const void* toks[6] = {weight_decay, receptance, key, value, removal, replacement};
  if (sh.tok_elems() > 0) {
    for (const void* p : toks)
      if (!p) return WKV7_ERR_NULL_POINTER;
    if (!state && sh.ckpt_elems() > 0) return WKV7_ERR_NULL_POINTER;
    if (!removal_state || !output) return WKV7_ERR_NULL_POINTER;
  }
  if (sh.state_elems() > 0) {
    if (use_initial_state && !initial_state) return WKV7_ERR_NULL_POINTER;
    if (return_final_state && !final_state) return WKV7_ERR_NULL_POINTER;
  }
  const uintptr_t ta = dtype == WKV7_DTYPE_BF16 ? 8 : 16;
  for (const void* p : toks)
    if (!aligned(p, ta)) return WKV7_ERR_ALIGNMENT;
  if (!aligned(output, ta) || !aligned(state, 16) || !aligned(removal_state, 16) ||
      !aligned(initial_state, 16) || !aligned(final_state, 16))
    return WKV7_ERR_ALIGNMENT;
  std::vector<Range> ins;
  for (const void* p : toks) ins.push_back({p, tok});
  if (use_initial_state) ins.push_back({initial_state, st});
  std::vector<Range> outs = {{state, sh.ckpt_elems() * 4},
                             {removal_state, sh.tok_elems() * 4},
                             {output, tok}};
  if (return_final_state) outs.push_back({final_state, st});
  if (any_overlap(outs, ins)) return WKV7_ERR_OVERLAP;
  if (sh.state_elems() == 0) return WKV7_OK;

  wkv7::ForwardDesc d;
  d.dtype = static_cast<wkv7::Dtype>(dtype);
  d.B = static_cast<int>(batch_size);
  d.T = static_cast<int>(context_len);
  d.H = static_cast<int>(num_heads);
  d.C = static_cast<int>(chunk_len);
  d.w = weight_decay; d.r = receptance; d.k = key; d.v = value; d.a = removal; d.b = replacement;
  d.s0 = use_initial_state ? initial_state : nullptr;
  d.ckpt = state;
  d.sa = removal_state;
  d.y = output;
  d.sT = return_final_state ? final_state : nullptr;
  d.kc = kc;
  return hip_status(wkv7::launch_forward(d, static_cast<hipStream_t>(stream)));
}

int wkv7_backward(const void* weight_decay, const void* receptance, const void* key,
                  const void* value, const void* removal, const void* replacement,
                  const float* state, const float* removal_state, const void* output_grad,
                  const float* final_state_grad, int64_t batch_size, int64_t context_len,
                  int64_t num_heads, int64_t head_size, int64_t chunk_len, int dtype,
                  int use_final_state_grad, int write_initial_state_grad,
                  void* weight_decay_grad, void* receptance_grad, void* key_grad,
                  void* value_grad, void* removal_grad, void* replacement_grad,
                  float* initial_state_grad, void* stream) {
  return wkv7_backward_ex(weight_decay, receptance, key, value, removal, replacement, state,
                          removal_state, output_grad, final_state_grad, batch_size, context_len,
                          num_heads, head_size, chunk_len, dtype, use_final_state_grad,
                          write_initial_state_grad, weight_decay_grad, receptance_grad,
                          key_grad, value_grad, removal_grad, replacement_grad,
                          initial_state_grad, nullptr, stream);
}

int wkv7_backward_ex(const void* weight_decay, const void* receptance, const void* key,
                     const void* value, const void* removal, const void* replacement,
                     const float* state, const float* removal_state, const void* output_grad,
                     const float* final_state_grad, int64_t batch_size, int64_t context_len,
                     int64_t num_heads, int64_t head_size, int64_t chunk_len, int dtype,
                     int use_final_state_grad, int write_initial_state_grad,
                     void* weight_decay_grad, void* receptance_grad, void* key_grad,
                     void* value_grad, void* removal_grad, void* replacement_grad,
                     float* initial_state_grad, const wkv7_options* options, void* stream) {
  wkv7::KernelChoice kc;
  if (int rc = kernel_choice(options, &kc)) return rc;
  if (int rc = check_shape(batch_size, context_len, num_heads, head_size, chunk_len, dtype))
    return rc;
  if (int rc = check_flag(use_final_state_grad)) return rc;
  if (int rc = check_flag(write_initial_state_grad)) return rc;
  const Shape sh{batch_size, context_len, num_heads, chunk_len};
  const int64_t tok = sh.tok_elems() * elem_bytes(dtype);
  const int64_t st = sh.state_elems() * 4;
  const void* toks[7] = {weight_decay, receptance, key, value, removal, replacement, output_grad};
  void* grads[6] = {weight_decay_grad, receptance_grad, key_grad, value_grad, removal_grad,
                    replacement_grad};
  if (sh.tok_elems() > 0) {
    for (const void* p : toks)
      if (!p) return WKV7_ERR_NULL_POINTER;
    for (const void* p : grads)
      if (!p) return WKV7_ERR_NULL_POINTER;
    if (!state || !removal_state) return WKV7_ERR_NULL_POINTER;
  }
  if (sh.state_elems() > 0) {
    if (use_final_state_grad && !final_state_grad) return WKV7_ERR_NULL_POINTER;
    if (write_initial_state_grad && !initial_state_grad) return WKV7_ERR_NULL_POINTER;
  }
  const uintptr_t ta = dtype == WKV7_DTYPE_BF16 ? 8 : 16;
  for (const void* p : toks)
    if (!aligned(p, ta)) return WKV7_ERR_ALIGNMENT;
  for (const void* p : grads)
    if (!aligned(p, ta)) return WKV7_ERR_ALIGNMENT;
  if (!aligned(state, 16) || !aligned(removal_state, 16) || !aligned(final_state_grad, 16) ||
      !aligned(initial_state_grad, 16))
    return WKV7_ERR_ALIGNMENT;
  std::vector<Range> ins;
  for (const void* p : toks) ins.push_back({p, tok});
  ins.push_back({state, sh.ckpt_elems() * 4});
  ins.push_back({removal_state, sh.tok_elems() * 4});
  if (use_final_state_grad) ins.push_back({final_state_grad, st});
  std::vector<Range> outs;
  for (void* p : grads) outs.push_back({p, tok});
  if (write_initial_state_grad) outs.push_back({initial_state_grad, st});
  if (any_overlap(outs, ins)) return WKV7_ERR_OVERLAP;
  if (sh.state_elems() == 0) return WKV7_OK;

  wkv7::BackwardDesc d;
  d.dtype = static_cast<wkv7::Dtype>(dtype);
  d.B = static_cast<int>(batch_size);
  d.T = static_cast<int>(context_len);
  d.H = static_cast<int>(num_heads);
  d.C = static_cast<int>(chunk_len);
  d.w = weight_decay; d.r = receptance; d.k = key; d.v = value; d.a = removal; d.b = replacement;
  d.ckpt = state;
  d.sa = removal_state;
  d.dy = output_grad;
  d.dsT = use_final_state_grad ? final_state_grad : nullptr;
  d.dw = weight_decay_grad; d.dr = receptance_grad; d.dk = key_grad; d.dv = value_grad;
  d.da = removal_grad; d.db = replacement_grad;
  d.ds0 = write_initial_state_grad ? initial_state_grad : nullptr;
  d.kc = kc;
  return hip_status(wkv7::launch_backward(d, static_cast<hipStream_t>(stream)));
}

// ---- Burn backend trait mirrors: fixed flags exactly as the reference's
// CubeBackend impls pass them.

// wkv7_pretrain/forward.rs:19-46: use_initial_state = false, return_final_state = false
int wkv7_pretrain_forward(const void* w, const void* r, const void* k, const void* v,
                          const void* a, const void* b, int64_t B, int64_t T, int64_t H,
                          int64_t N, int64_t C, int dtype, float* state, float* removal_state,
                          void* output, void* stream) {
  return wkv7_forward(w, r, k, v, a, b, nullptr, B, T, H, N, C, dtype, 0, 0, state,
                      removal_state, output, nullptr, stream);
}

// wkv7_pretrain/forward.rs:48-84: use_final_state_grad = false, write_initial_state_grad = false
int wkv7_pretrain_backward(const void* w, const void* r, const void* k, const void* v,
                           const void* a, const void* b, const float* state,
                           const float* removal_state, const void* output_grad, int64_t B,
                           int64_t T, int64_t H, int64_t N, int64_t C, int dtype, void* dw,
                           void* dr, void* dk, void* dv, void* da, void* db, void* stream) {
  return wkv7_backward(w, r, k, v, a, b, state, removal_state, output_grad, nullptr, B, T, H, N,
                       C, dtype, 0, 0, dw, dr, dk, dv, da, db, nullptr, stream);
}

// wkv7_statepass/forward.rs:17-39: use_initial_state = true, return_final_state = true
int wkv7_statepass_forward(const void* w, const void* r, const void* k, const void* v,
                           const void* a, const void* b, const float* initial_state, int64_t B,
                           int64_t T, int64_t H, int64_t N, int64_t C, int dtype, float* state,
                           float* removal_state, void* output, float* final_state,
                           void* stream) {
  return wkv7_forward(w, r, k, v, a, b, initial_state, B, T, H, N, C, dtype, 1, 1, state,
                      removal_state, output, final_state, stream);
}

// wkv7_statepass/forward.rs:41-69: use_final_state_grad = true, write_initial_state_grad = true
int wkv7_statepass_backward(const void* w, const void* r, const void* k, const void* v,
                            const void* a, const void* b, const float* state,
                            const float* removal_state, const void* output_grad,
                            const float* final_state_grad, int64_t B, int64_t T, int64_t H,
                            int64_t N, int64_t C, int dtype, void* dw, void* dr, void* dk,
                            void* dv, void* da, void* db, float* initial_state_grad,
                            void* stream) {
  return wkv7_backward(w, r, k, v, a, b, state, removal_state, output_grad, final_state_grad, B,
                       T, H, N, C, dtype, 1, 1, dw, dr, dk, dv, da, db, initial_state_grad,
                       stream);
}

// wkv7_statetune/forward.rs:29-40: use_initial_state = true, return_final_state = false
int wkv7_statetune_forward(const void* w, const void* r, const void* k, const void* v,
                           const void* a, const void* b, const float* initial_state, int64_t B,
                           int64_t T, int64_t H, int64_t N, int64_t C, int dtype, float* state,
                           float* removal_state, void* output, void* stream) {
  return wkv7_forward(w, r, k, v, a, b, initial_state, B, T, H, N, C, dtype, 1, 0, state,
                      removal_state, output, nullptr, stream);
}

// wkv7_statetune/forward.rs:61-75: use_final_state_grad = false, write_initial_state_grad = true
int wkv7_statetune_backward(const void* w, const void* r, const void* k, const void* v,
                            const void* a, const void* b, const float* state,
                            const float* removal_state, const void* output_grad, int64_t B,
                            int64_t T, int64_t H, int64_t N, int64_t C, int dtype, void* dw,
                            void* dr, void* dk, void* dv, void* da, void* db,
                            float* initial_state_grad, void* stream) {
  return wkv7_backward(w, r, k, v, a, b, state, removal_state, output_grad, nullptr, B, T, H, N,
                       C, dtype, 0, 1, dw, dr, dk, dv, da, db, initial_state_grad, stream);
}

int wkv7_infer_forward(const void* weight_decay, const void* receptance, const void* key,
                       const void* value, const void* removal, const void* replacement,
                       const int32_t* batch_ids, void* state, const void* context_mask,
                       const int32_t* elapsed_t, int64_t active_batch_size, int64_t context_len,
                       int64_t num_heads, int64_t head_size, int64_t full_batch_size, int dtype,
                       int state_dtype, int use_dither, void* output, void* stream) {
  if (int rc = check_dtype(dtype)) return rc;
  if (int rc = check_dtype(state_dtype)) return rc;
  // a bf16 state is the reference's kernel at element type bf16: every
  // operand is bf16 too
  if (state_dtype == WKV7_DTYPE_BF16 && dtype != WKV7_DTYPE_BF16) return WKV7_ERR_DTYPE;
  if (head_size != kN) return WKV7_ERR_HEAD_SIZE;
  if (active_batch_size < 0 || context_len < 0 || num_heads < 0 || full_batch_size < 0 ||
      active_batch_size > kMaxGridDim || num_heads > kMaxGridDim || context_len > INT32_MAX ||
      full_batch_size > INT32_MAX || active_batch_size > full_batch_size)
    return WKV7_ERR_SHAPE;
  if (!product_fits({active_batch_size, context_len, num_heads, kN, 4}) ||
      !product_fits({full_batch_size, num_heads, kN * kN, 4}))
    return WKV7_ERR_SHAPE;
  if (int rc = check_flag(use_dither)) return rc;
  // the reference dithers only when the element type is not f32 (host.rs:157)
  if (use_dither && state_dtype != WKV7_DTYPE_BF16) return WKV7_ERR_FLAGS;
  const int64_t toks_n = active_batch_size * context_len * num_heads * kN;
  const int64_t tok = toks_n * elem_bytes(dtype);
  const int64_t st = full_batch_size * num_heads * kN * kN * elem_bytes(state_dtype);
  const void* toks[6] = {weight_decay, receptance, key, value, removal, replacement};
  if (toks_n > 0) {
    for (const void* p : toks)
      if (!p) return WKV7_ERR_NULL_POINTER;
    if (!output) return WKV7_ERR_NULL_POINTER;
  }
  if (active_batch_size > 0 && num_heads > 0) {
    if (!batch_ids || !state) return WKV7_ERR_NULL_POINTER;
    if (use_dither && !elapsed_t) return WKV7_ERR_NULL_POINTER;
  }
  const uintptr_t ta = dtype == WKV7_DTYPE_BF16 ? 8 : 16;
  for (const void* p : toks)
    if (!aligned(p, ta)) return WKV7_ERR_ALIGNMENT;
  if (!aligned(output, ta) || !aligned(state, 16) || !aligned(batch_ids, 4) ||
      !aligned(elapsed_t, 4) || !aligned(context_mask, dtype == WKV7_DTYPE_BF16 ? 2 : 4))
    return WKV7_ERR_ALIGNMENT;
  std::vector<Range> ins;
  for (const void* p : toks) ins.push_back({p, tok});
  ins.push_back({batch_ids, active_batch_size * 4});
  ins.push_back({context_mask, context_mask ? active_batch_size * context_len * elem_bytes(dtype) : 0});
  ins.push_back({elapsed_t, elapsed_t ? full_batch_size * 4 : 0});
  // the state is updated in place: it may not overlap the inputs or the output
  std::vector<Range> outs = {{output, tok}, {state, st}};
  if (any_overlap(outs, ins)) return WKV7_ERR_OVERLAP;
  if (active_batch_size == 0 || num_heads == 0) return WKV7_OK;

  wkv7::InferDesc d;
  d.dtype = static_cast<wkv7::Dtype>(dtype);
  d.state_dtype = static_cast<wkv7::Dtype>(state_dtype);
  d.Ba = static_cast<int>(active_batch_size);
  d.T = static_cast<int>(context_len);
  d.H = static_cast<int>(num_heads);
  d.full_batch = static_cast<int>(full_batch_size);
  d.w = weight_decay; d.r = receptance; d.k = key; d.v = value; d.a = removal; d.b = replacement;
  d.batch_ids = batch_ids;
  d.state = state;
  d.context_mask = context_mask;
  d.elapsed_t = elapsed_t;
  d.use_dither = use_dither;
  d.y = output;
  return hip_status(wkv7::launch_infer(d, static_cast<hipStream_t>(stream)));
}

}  // extern "C"
