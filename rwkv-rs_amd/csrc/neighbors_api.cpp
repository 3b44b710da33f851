// C ABI of the ops beside the WKV7 operator: argument validation and
// dispatch. Every check happens on the host before any HIP call, so a bad
// call returns a wkv7_status code instead of launching a kernel whose grid or
// indexing does not match its buffers.
#include "../../include/rwkv_neighbors.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <initializer_list>
#include <vector>

#include "neighbors_launch.hpp"
#include "wkv7_launch.hpp"

static_assert(rwkv_nb::kReadoutScratchBytes == RWKV_READOUT_SCRATCH_BYTES,
              "the scratch array size the header states");

namespace {

constexpr int64_t kMaxGridY = 65535;
constexpr int64_t kMaxGridX = INT32_MAX;

struct Range {
  const void* p;
  int64_t bytes;
};

bool overlaps(const Range& x, const Range& y) {
  if (!x.p || !y.p || x.bytes <= 0 || y.bytes <= 0) return false;
  const auto a0 = reinterpret_cast<uintptr_t>(x.p), b0 = reinterpret_cast<uintptr_t>(y.p);
  return a0 < b0 + static_cast<uintptr_t>(y.bytes) && b0 < a0 + static_cast<uintptr_t>(x.bytes);
}

bool any_overlap(const std::vector<Range>& outs, const std::vector<Range>& ins) {
  for (size_t i = 0; i < outs.size(); ++i) {
    for (size_t j = i + 1; j < outs.size(); ++j)
      if (overlaps(outs[i], outs[j])) return true;
    for (const Range& in : ins)
      if (overlaps(outs[i], in)) return true;
  }
  return false;
}

bool valid_dtype(int d) { return d == WKV7_DTYPE_F32 || d == WKV7_DTYPE_BF16; }

// the product of the factors fits int64 (no wrap-around)
bool product_fits(std::initializer_list<int64_t> factors) {
  int64_t acc = 1;
  for (int64_t f : factors)
    if (__builtin_mul_overflow(acc, f, &acc)) return false;
  return true;
}
// Every byte count these checks and the workspace sizes form is at most
// elements x 8 x (sums per element) of one of the shapes below, so shapes
// for which those products fit int64 never overflow.
bool mix_sizes_fit(int64_t rows, int64_t C, int64_t full_batch) {
  return product_fits({rows, C, 8, rwkv_nb::kMaxMixes}) && product_fits({full_batch, C, 8});
}
bool head_rows_fit(int64_t rows, int64_t H, int64_t sums) {
  return product_fits({rows, H, 64, 8, sums});
}
int64_t esize(int d) { return d == WKV7_DTYPE_BF16 ? 2 : 4; }
bool aligned_for(const void* p, int d) {
  return (reinterpret_cast<uintptr_t>(p) % (d == WKV7_DTYPE_BF16 ? 8 : 16)) == 0;
}

// shared shape and pointer checks of the token-shift mix
int check_shift_mix(const void* x, const void* shift, const int32_t* batch_ids,
                    const void* mask, const float* scales, int64_t K, int64_t B, int64_t T,
                    int64_t C, int64_t full_batch, int dtype, int out_dtype) {
  if (!valid_dtype(dtype) || !valid_dtype(out_dtype)) return WKV7_ERR_DTYPE;
  if (K < 0 || K > rwkv_nb::kMaxMixes) return WKV7_ERR_SHAPE;
  if (B < 0 || T < 0 || C <= 0 || C % 4 != 0 || full_batch < 0) return WKV7_ERR_SHAPE;
  if (B > kMaxGridY || C / rwkv_nb::kMixColsPerBlock + 1 > kMaxGridY) return WKV7_ERR_SHAPE;
  if (T > 0 && B > INT64_MAX / T) return WKV7_ERR_SHAPE;
  const int64_t rows = B * T;
  if (!mix_sizes_fit(rows, C, full_batch)) return WKV7_ERR_SHAPE;
  if (rwkv_nb::mix_row_blocks(rows) > kMaxGridX) return WKV7_ERR_SHAPE;
  if (rows > 0 && !x) return WKV7_ERR_NULL_POINTER;
  if (K > 0 && !scales) return WKV7_ERR_NULL_POINTER;
  if (!batch_ids && full_batch < B) return WKV7_ERR_SHAPE;
  if ((x && !aligned_for(x, dtype)) || (shift && !aligned_for(shift, dtype)) ||
      (scales && !aligned_for(scales, WKV7_DTYPE_F32)) ||
      (reinterpret_cast<uintptr_t>(mask) % esize(dtype)) != 0)
    return WKV7_ERR_ALIGNMENT;
  return WKV7_OK;
}

int64_t shift_mix_workspace(int64_t K, int64_t B, int64_t T, int64_t C) {
  return rwkv_nb::mix_row_blocks(B * T) * K * C * 4;
}

int check_readout(const void* y, const void* r, const void* k, const void* v, const void* gate,
                  const float* bonus, const float* weight, const float* bias, float eps,
                  int64_t rows, int64_t H, int64_t N, int dtype, int act_dtype) {
  if (!valid_dtype(dtype) || !valid_dtype(act_dtype)) return WKV7_ERR_DTYPE;
  if (N != 64) return WKV7_ERR_HEAD_SIZE;
  if (rows < 0 || H <= 0 || H > kMaxGridY) return WKV7_ERR_SHAPE;
  if (!head_rows_fit(rows, H, rwkv_nb::kReadoutSums)) return WKV7_ERR_SHAPE;
  if (rwkv_nb::readout_row_blocks(rows) > kMaxGridX) return WKV7_ERR_SHAPE;
  if (!(eps >= 0.f) || !std::isfinite(eps)) return WKV7_ERR_SHAPE;
  if (!bonus || !weight || !bias) return WKV7_ERR_NULL_POINTER;
  if (rows > 0 && (!y || !r || !k || !v || !gate)) return WKV7_ERR_NULL_POINTER;
  for (const void* p : {y, r, k, v})
    if (p && !aligned_for(p, dtype)) return WKV7_ERR_ALIGNMENT;
  if (gate && !aligned_for(gate, act_dtype)) return WKV7_ERR_ALIGNMENT;
  for (const float* p : {bonus, weight, bias})
    if (!aligned_for(p, WKV7_DTYPE_F32)) return WKV7_ERR_ALIGNMENT;
  return WKV7_OK;
}

// shared shape and pointer checks of the weight preparation's end; the
// value residual is on exactly when its bias is given
int check_prepare(const void* key, const void* value, const void* value_first, const void* lr,
                  const void* wd, const void* vr, const float* lr_bias, const float* wd_bias,
                  const float* vr_bias, const float* ka, const float* kk, int64_t rows, int64_t H,
                  int64_t N, int dtype, int out_dtype) {
  if (!valid_dtype(dtype) || !valid_dtype(out_dtype)) return WKV7_ERR_DTYPE;
  if (N != 64) return WKV7_ERR_HEAD_SIZE;
  if (rows < 0 || H <= 0 || H > kMaxGridY) return WKV7_ERR_SHAPE;
  if (!head_rows_fit(rows, H, rwkv_nb::kPrepareSums)) return WKV7_ERR_SHAPE;
  if (rwkv_nb::prepare_row_blocks(rows) > kMaxGridX) return WKV7_ERR_SHAPE;
  if (!lr_bias || !wd_bias || !ka || !kk) return WKV7_ERR_NULL_POINTER;
  const bool res = vr_bias != nullptr;
  if (!res && (value_first || vr)) return WKV7_ERR_SHAPE;  // a residual input without its bias
  if (rows > 0 && (!key || !value || !lr || !wd || (res && (!value_first || !vr))))
    return WKV7_ERR_NULL_POINTER;
  for (const void* p : {key, value, value_first, lr, wd, vr})
    if (p && !aligned_for(p, dtype)) return WKV7_ERR_ALIGNMENT;
  for (const float* p : {lr_bias, wd_bias, vr_bias, ka, kk})
    if (p && !aligned_for(p, WKV7_DTYPE_F32)) return WKV7_ERR_ALIGNMENT;
  return WKV7_OK;
}

int64_t prepare_workspace(int64_t rows, int64_t H) {
  return rwkv_nb::prepare_row_blocks(rows) * rwkv_nb::kPrepareSums * H * 64 * 4;
}

rwkv_nb::PrepareArgs prepare_args(const void* key, const void* value, const void* value_first,
                                  const void* lr, const void* wd, const void* vr,
                                  const float* lr_bias, const float* wd_bias,
                                  const float* vr_bias, const float* ka, const float* kk,
                                  int64_t rows, int64_t H, int dtype, int out_dtype) {
  rwkv_nb::PrepareArgs a{};
  a.key = key;
  a.value = value;
  a.value_first = value_first;
  a.lr = lr;
  a.wd = wd;
  a.vr = vr;
  a.lr_bias = lr_bias;
  a.wd_bias = wd_bias;
  a.vr_bias = vr_bias;
  a.key_replacement = ka;
  a.key_removal = kk;
  a.rows = rows;
  a.H = H;
  a.in_bf16 = dtype == WKV7_DTYPE_BF16;
  a.out_bf16 = out_dtype == WKV7_DTYPE_BF16;
  a.residual = vr_bias != nullptr;
  return a;
}

int64_t readout_workspace(int64_t rows, int64_t H) {
  return rwkv_nb::readout_row_blocks(rows) * rwkv_nb::kReadoutSums * H * 64 * 4;
}

}  // namespace

extern "C" {

int64_t rwkv_token_shift_mix_workspace_bytes(int64_t num_mixes, int64_t batch_size,
                                             int64_t context_len, int64_t embedded_dim) {
  if (num_mixes < 0 || num_mixes > rwkv_nb::kMaxMixes || batch_size < 0 || context_len < 0 ||
      embedded_dim <= 0 || embedded_dim % 4 != 0)
    return -1;
  if (context_len > 0 && batch_size > INT64_MAX / context_len) return -1;
  if (!mix_sizes_fit(batch_size * context_len, embedded_dim, 0)) return -1;
  return shift_mix_workspace(num_mixes, batch_size, context_len, embedded_dim);
}

int rwkv_token_shift_mix_forward(const void* embedded_context, const void* embedded_token_shift,
                                 const int32_t* batch_ids, const void* context_mask,
                                 const float* scales, int64_t num_mixes, int64_t batch_size,
                                 int64_t context_len, int64_t embedded_dim,
                                 int64_t full_batch_size, int dtype, int out_dtype,
                                 void* const* mixes, void* token_shifted_diff,
                                 void* next_token_shift, void* stream) {
  const int64_t K = num_mixes, B = batch_size, T = context_len, C = embedded_dim;
  if (int rc = check_shift_mix(embedded_context, embedded_token_shift, batch_ids, context_mask,
                               scales, K, B, T, C, full_batch_size, dtype, out_dtype))
    return rc;
  if (K > 0 && !mixes) return WKV7_ERR_NULL_POINTER;
  const int64_t rows = B * T;
  const int64_t out_bytes = rows * C * esize(out_dtype);
  std::vector<Range> outs, ins = {{embedded_context, rows * C * esize(dtype)},
                                  {batch_ids, B * 4},
                                  {context_mask, rows * esize(dtype)},
                                  {scales, K * C * 4}};
  for (int64_t i = 0; i < K; ++i) {
    if (!mixes[i]) return WKV7_ERR_NULL_POINTER;
    if (!aligned_for(mixes[i], out_dtype)) return WKV7_ERR_ALIGNMENT;
    outs.push_back({mixes[i], out_bytes});
  }
  if (token_shifted_diff) {
    if (!aligned_for(token_shifted_diff, out_dtype)) return WKV7_ERR_ALIGNMENT;
    outs.push_back({token_shifted_diff, out_bytes});
  }
  const int64_t shift_bytes = full_batch_size * C * esize(dtype);
  if (next_token_shift) {
    if (!aligned_for(next_token_shift, dtype)) return WKV7_ERR_ALIGNMENT;
    // the shift buffer itself may be updated in place, but not overlap partly
    if (next_token_shift != embedded_token_shift &&
        overlaps({next_token_shift, shift_bytes}, {embedded_token_shift, shift_bytes}))
      return WKV7_ERR_OVERLAP;
    outs.push_back({next_token_shift, shift_bytes});
  }
  std::vector<Range> ins_all = ins;
  if (next_token_shift != embedded_token_shift) ins_all.push_back({embedded_token_shift, shift_bytes});
  if (any_overlap(outs, ins_all)) return WKV7_ERR_OVERLAP;
  if (next_token_shift == embedded_token_shift && embedded_token_shift) {
    for (size_t i = 0; i + 1 < outs.size(); ++i)
      if (overlaps(outs[i], {embedded_token_shift, shift_bytes})) return WKV7_ERR_OVERLAP;
  }

  rwkv_nb::ShiftMixArgs a{};
  a.x = embedded_context;
  a.shift = embedded_token_shift;
  a.batch_ids = batch_ids;
  a.mask = context_mask;
  a.scales = scales;
  a.batch = B;
  a.T = T;
  a.C = C;
  a.full_batch = full_batch_size;
  a.num_mixes = static_cast<int>(K);
  a.x_bf16 = dtype == WKV7_DTYPE_BF16;
  a.out_bf16 = out_dtype == WKV7_DTYPE_BF16;
  for (int64_t i = 0; i < K; ++i) a.mixes[i] = mixes[i];
  a.diff = token_shifted_diff;
  a.next_shift = next_token_shift;
  return wkv7::hip_status(
      rwkv_nb::launch_shift_mix_forward(a, static_cast<hipStream_t>(stream)));
}

int rwkv_token_shift_mix_backward(const void* embedded_context, const void* embedded_token_shift,
                                  const int32_t* batch_ids, const void* context_mask,
                                  const float* scales, int64_t num_mixes, int64_t batch_size,
                                  int64_t context_len, int64_t embedded_dim,
                                  int64_t full_batch_size, int dtype, int out_dtype,
                                  const void* const* mix_grads,
                                  const void* token_shifted_diff_grad,
                                  void* embedded_context_grad, float* embedded_token_shift_grad,
                                  float* scales_grad, void* workspace, int64_t workspace_bytes,
                                  void* stream) {
  const int64_t K = num_mixes, B = batch_size, T = context_len, C = embedded_dim;
  if (int rc = check_shift_mix(embedded_context, embedded_token_shift, batch_ids, context_mask,
                               scales, K, B, T, C, full_batch_size, dtype, out_dtype))
    return rc;
  const int64_t rows = B * T;
  if (K > 0 && (!mix_grads || !scales_grad)) return WKV7_ERR_NULL_POINTER;
  if (rows > 0 && !embedded_context_grad) return WKV7_ERR_NULL_POINTER;
  const int64_t need = shift_mix_workspace(K, B, T, C);
  if (need > 0 && (!workspace || workspace_bytes < need)) return WKV7_ERR_SHAPE;
  if (workspace && !aligned_for(workspace, WKV7_DTYPE_F32)) return WKV7_ERR_ALIGNMENT;
  const int64_t g_bytes = rows * C * esize(out_dtype);
  std::vector<Range> ins = {{embedded_context, rows * C * esize(dtype)},
                            {embedded_token_shift, full_batch_size * C * esize(dtype)},
                            {batch_ids, B * 4},
                            {context_mask, rows * esize(dtype)},
                            {scales, K * C * 4},
                            {token_shifted_diff_grad, token_shifted_diff_grad ? g_bytes : 0}};
  if (token_shifted_diff_grad && !aligned_for(token_shifted_diff_grad, out_dtype))
    return WKV7_ERR_ALIGNMENT;
  for (int64_t i = 0; i < K; ++i) {
    if (!mix_grads[i]) return WKV7_ERR_NULL_POINTER;
    if (!aligned_for(mix_grads[i], out_dtype)) return WKV7_ERR_ALIGNMENT;
    ins.push_back({mix_grads[i], g_bytes});
  }
  if ((embedded_context_grad && !aligned_for(embedded_context_grad, dtype)) ||
      (embedded_token_shift_grad && !aligned_for(embedded_token_shift_grad, WKV7_DTYPE_F32)) ||
      (scales_grad && !aligned_for(scales_grad, WKV7_DTYPE_F32)))
    return WKV7_ERR_ALIGNMENT;
  const std::vector<Range> outs = {{embedded_context_grad, rows * C * esize(dtype)},
                                   {embedded_token_shift_grad, full_batch_size * C * 4},
                                   {scales_grad, K * C * 4},
                                   {workspace, need}};
  if (any_overlap(outs, ins)) return WKV7_ERR_OVERLAP;

  rwkv_nb::ShiftMixArgs a{};
  a.x = embedded_context;
  a.shift = embedded_token_shift;
  a.batch_ids = batch_ids;
  a.mask = context_mask;
  a.scales = scales;
  a.batch = B;
  a.T = T;
  a.C = C;
  a.full_batch = full_batch_size;
  a.num_mixes = static_cast<int>(K);
  a.x_bf16 = dtype == WKV7_DTYPE_BF16;
  a.out_bf16 = out_dtype == WKV7_DTYPE_BF16;
  for (int64_t i = 0; i < K; ++i) a.mix_grads[i] = mix_grads[i];
  a.diff_grad = token_shifted_diff_grad;
  a.x_grad = embedded_context_grad;
  a.shift_grad = embedded_token_shift_grad;
  a.scales_grad = scales_grad;
  a.workspace = static_cast<float*>(workspace);
  return wkv7::hip_status(
      rwkv_nb::launch_shift_mix_backward(a, static_cast<hipStream_t>(stream)));
}

int64_t rwkv_gated_readout_workspace_bytes(int64_t rows, int64_t num_heads, int64_t head_size) {
  if (rows < 0 || num_heads <= 0 || head_size != 64) return -1;
  if (!head_rows_fit(rows, num_heads, rwkv_nb::kReadoutSums)) return -1;
  return readout_workspace(rows, num_heads);
}

int rwkv_gated_readout_forward(const void* wkv7_output, const void* receptance,
                               const void* replacement_key, const void* value, const void* gate,
                               const float* receptance_key_bonus, const float* group_norm_weight,
                               const float* group_norm_bias, float epsilon, int64_t rows,
                               int64_t num_heads, int64_t head_size, int dtype, int act_dtype,
                               void* output, void* stream) {
  if (int rc = check_readout(wkv7_output, receptance, replacement_key, value, gate,
                             receptance_key_bonus, group_norm_weight, group_norm_bias, epsilon,
                             rows, num_heads, head_size, dtype, act_dtype))
    return rc;
  const int64_t C = num_heads * 64;
  if (rows > 0 && !output) return WKV7_ERR_NULL_POINTER;
  if (output && !aligned_for(output, act_dtype)) return WKV7_ERR_ALIGNMENT;
  const int64_t op = rows * C * esize(dtype), act = rows * C * esize(act_dtype);
  if (any_overlap({{output, act}},
                  {{wkv7_output, op}, {receptance, op}, {replacement_key, op}, {value, op},
                   {gate, act}, {receptance_key_bonus, C * 4}, {group_norm_weight, C * 4},
                   {group_norm_bias, C * 4}}))
    return WKV7_ERR_OVERLAP;
  rwkv_nb::ReadoutArgs a{};
  a.y = wkv7_output;
  a.r = receptance;
  a.k = replacement_key;
  a.v = value;
  a.gate = gate;
  a.bonus = receptance_key_bonus;
  a.weight = group_norm_weight;
  a.bias = group_norm_bias;
  a.eps = epsilon;
  a.rows = rows;
  a.H = num_heads;
  a.op_bf16 = dtype == WKV7_DTYPE_BF16;
  a.act_bf16 = act_dtype == WKV7_DTYPE_BF16;
  a.out = output;
  return wkv7::hip_status(rwkv_nb::launch_readout_forward(a, static_cast<hipStream_t>(stream)));
}

}  // extern "C"

namespace {

// Checks and launch of the gated readout backward, shared by the entry point
// that takes a workspace and the one that uses the library's scratch array.
// With `scratch` set, `workspace` is ignored: the checks run first and the
// scratch array's device address is looked up only for a valid call.
int readout_backward(const void* wkv7_output, const void* receptance,
                     const void* replacement_key, const void* value, const void* gate,
                     const float* receptance_key_bonus, const float* group_norm_weight,
                     const float* group_norm_bias, float epsilon, int64_t rows,
                     int64_t num_heads, int64_t head_size, int dtype, int act_dtype,
                     const void* output_grad, void* wkv7_output_grad, void* receptance_grad,
                     void* replacement_key_grad, void* value_grad, void* gate_grad,
                     float* receptance_key_bonus_grad, float* group_norm_weight_grad,
                     float* group_norm_bias_grad, void* workspace, int64_t workspace_bytes,
                     bool scratch, void* stream) {
  if (int rc = check_readout(wkv7_output, receptance, replacement_key, value, gate,
                             receptance_key_bonus, group_norm_weight, group_norm_bias, epsilon,
                             rows, num_heads, head_size, dtype, act_dtype))
    return rc;
  const int64_t C = num_heads * 64;
  if (!receptance_key_bonus_grad || !group_norm_weight_grad || !group_norm_bias_grad)
    return WKV7_ERR_NULL_POINTER;
  if (rows > 0 && (!output_grad || !wkv7_output_grad || !receptance_grad ||
                   !replacement_key_grad || !value_grad || !gate_grad))
    return WKV7_ERR_NULL_POINTER;
  const int64_t need = readout_workspace(rows, num_heads);
  if (scratch) {
    if (need > rwkv_nb::kReadoutScratchBytes) return WKV7_ERR_SCRATCH_LIMIT;
    workspace = nullptr;
  } else if (need > 0 && (!workspace || workspace_bytes < need)) {
    return WKV7_ERR_SHAPE;
  }
  for (const void* p : {wkv7_output_grad, receptance_grad, replacement_key_grad, value_grad})
    if (p && !aligned_for(p, dtype)) return WKV7_ERR_ALIGNMENT;
  for (const void* p : {output_grad, static_cast<const void*>(gate_grad)})
    if (p && !aligned_for(p, act_dtype)) return WKV7_ERR_ALIGNMENT;
  for (const void* p : {static_cast<const void*>(receptance_key_bonus_grad),
                        static_cast<const void*>(group_norm_weight_grad),
                        static_cast<const void*>(group_norm_bias_grad),
                        static_cast<const void*>(workspace)})
    if (p && !aligned_for(p, WKV7_DTYPE_F32)) return WKV7_ERR_ALIGNMENT;
  const int64_t op = rows * C * esize(dtype), act = rows * C * esize(act_dtype);
  if (any_overlap({{wkv7_output_grad, op}, {receptance_grad, op}, {replacement_key_grad, op},
                   {value_grad, op}, {gate_grad, act}, {receptance_key_bonus_grad, C * 4},
                   {group_norm_weight_grad, C * 4}, {group_norm_bias_grad, C * 4},
                   {workspace, need}},
                  {{wkv7_output, op}, {receptance, op}, {replacement_key, op}, {value, op},
                   {gate, act}, {receptance_key_bonus, C * 4}, {group_norm_weight, C * 4},
                   {group_norm_bias, C * 4}, {output_grad, act}}))
    return WKV7_ERR_OVERLAP;
  float* ws = static_cast<float*>(workspace);
  if (scratch && need > 0) {
    if (int rc = wkv7::hip_status(rwkv_nb::readout_scratch(&ws))) return rc;
  }
  rwkv_nb::ReadoutArgs a{};
  a.y = wkv7_output;
  a.r = receptance;
  a.k = replacement_key;
  a.v = value;
  a.gate = gate;
  a.bonus = receptance_key_bonus;
  a.weight = group_norm_weight;
  a.bias = group_norm_bias;
  a.eps = epsilon;
  a.rows = rows;
  a.H = num_heads;
  a.op_bf16 = dtype == WKV7_DTYPE_BF16;
  a.act_bf16 = act_dtype == WKV7_DTYPE_BF16;
  a.out_grad = output_grad;
  a.y_grad = wkv7_output_grad;
  a.r_grad = receptance_grad;
  a.k_grad = replacement_key_grad;
  a.v_grad = value_grad;
  a.gate_grad = gate_grad;
  a.bonus_grad = receptance_key_bonus_grad;
  a.weight_grad = group_norm_weight_grad;
  a.bias_grad = group_norm_bias_grad;
  a.workspace = ws;
  return wkv7::hip_status(rwkv_nb::launch_readout_backward(a, static_cast<hipStream_t>(stream)));
}

}  // namespace

extern "C" {

int rwkv_gated_readout_backward(const void* wkv7_output, const void* receptance,
                                const void* replacement_key, const void* value, const void* gate,
                                const float* receptance_key_bonus,
                                const float* group_norm_weight, const float* group_norm_bias,
                                float epsilon, int64_t rows, int64_t num_heads, int64_t head_size,
                                int dtype, int act_dtype, const void* output_grad,
                                void* wkv7_output_grad, void* receptance_grad,
                                void* replacement_key_grad, void* value_grad, void* gate_grad,
                                float* receptance_key_bonus_grad, float* group_norm_weight_grad,
                                float* group_norm_bias_grad, void* workspace,
                                int64_t workspace_bytes, void* stream) {
  return readout_backward(wkv7_output, receptance, replacement_key, value, gate,
                          receptance_key_bonus, group_norm_weight, group_norm_bias, epsilon,
                          rows, num_heads, head_size, dtype, act_dtype, output_grad,
                          wkv7_output_grad, receptance_grad, replacement_key_grad, value_grad,
                          gate_grad, receptance_key_bonus_grad, group_norm_weight_grad,
                          group_norm_bias_grad, workspace, workspace_bytes, false, stream);
}

int rwkv_gated_readout_backward_noalloc(
    const void* wkv7_output, const void* receptance, const void* replacement_key,
    const void* value, const void* gate, const float* receptance_key_bonus,
    const float* group_norm_weight, const float* group_norm_bias, float epsilon, int64_t rows,
    int64_t num_heads, int64_t head_size, int dtype, int act_dtype, const void* output_grad,
    void* wkv7_output_grad, void* receptance_grad, void* replacement_key_grad, void* value_grad,
    void* gate_grad, float* receptance_key_bonus_grad, float* group_norm_weight_grad,
    float* group_norm_bias_grad, void* stream) {
  return readout_backward(wkv7_output, receptance, replacement_key, value, gate,
                          receptance_key_bonus, group_norm_weight, group_norm_bias, epsilon,
                          rows, num_heads, head_size, dtype, act_dtype, output_grad,
                          wkv7_output_grad, receptance_grad, replacement_key_grad, value_grad,
                          gate_grad, receptance_key_bonus_grad, group_norm_weight_grad,
                          group_norm_bias_grad, nullptr, 0, true, stream);
}

int64_t rwkv_weight_prepare_workspace_bytes(int64_t rows, int64_t num_heads, int64_t head_size) {
  if (rows < 0 || num_heads <= 0 || num_heads > kMaxGridY || head_size != 64) return -1;
  if (!head_rows_fit(rows, num_heads, rwkv_nb::kPrepareSums)) return -1;
  return prepare_workspace(rows, num_heads);
}

int rwkv_weight_prepare_forward(const void* key_precursor, const void* value_precursor,
                                const void* value_from_first_cell, const void* learning_rate_lora,
                                const void* weight_decay_lora, const void* value_residual_lora,
                                const float* learning_rate_bias, const float* weight_decay_bias,
                                const float* value_residual_bias, const float* key_replacement,
                                const float* key_removal, int64_t rows, int64_t num_heads,
                                int64_t head_size, int dtype, int out_dtype, void* weight_decay,
                                void* replacement_key, void* value, void* removal_key_normalized,
                                void* replacement, void* stream) {
  if (int rc = check_prepare(key_precursor, value_precursor, value_from_first_cell,
                             learning_rate_lora, weight_decay_lora, value_residual_lora,
                             learning_rate_bias, weight_decay_bias, value_residual_bias,
                             key_replacement, key_removal, rows, num_heads, head_size, dtype,
                             out_dtype))
    return rc;
  void* outs[] = {weight_decay, replacement_key, value, removal_key_normalized, replacement};
  for (void* p : outs) {
    if (rows > 0 && !p) return WKV7_ERR_NULL_POINTER;
    if (p && !aligned_for(p, out_dtype)) return WKV7_ERR_ALIGNMENT;
  }
  const int64_t C = num_heads * 64, in = rows * C * esize(dtype), out = rows * C * esize(out_dtype);
  std::vector<Range> o, i;
  for (void* p : outs) o.push_back({p, out});
  for (const void* p : {key_precursor, value_precursor, value_from_first_cell, learning_rate_lora,
                        weight_decay_lora, value_residual_lora})
    i.push_back({p, in});
  for (const float* p : {learning_rate_bias, weight_decay_bias, value_residual_bias,
                         key_replacement, key_removal})
    i.push_back({p, C * 4});
  if (any_overlap(o, i)) return WKV7_ERR_OVERLAP;
  rwkv_nb::PrepareArgs a = prepare_args(
      key_precursor, value_precursor, value_from_first_cell, learning_rate_lora,
      weight_decay_lora, value_residual_lora, learning_rate_bias, weight_decay_bias,
      value_residual_bias, key_replacement, key_removal, rows, num_heads, dtype, out_dtype);
  a.weight_decay = weight_decay;
  a.replacement_key = replacement_key;
  a.value_out = value;
  a.removal = removal_key_normalized;
  a.replacement = replacement;
  return wkv7::hip_status(rwkv_nb::launch_prepare_forward(a, static_cast<hipStream_t>(stream)));
}

int rwkv_weight_prepare_backward(
    const void* key_precursor, const void* value_precursor, const void* value_from_first_cell,
    const void* learning_rate_lora, const void* weight_decay_lora,
    const void* value_residual_lora, const float* learning_rate_bias,
    const float* weight_decay_bias, const float* value_residual_bias,
    const float* key_replacement, const float* key_removal, int64_t rows, int64_t num_heads,
    int64_t head_size, int dtype, int out_dtype, const void* weight_decay_grad,
    const void* replacement_key_grad, const void* value_grad,
    const void* removal_key_normalized_grad, const void* replacement_grad,
    void* key_precursor_grad, void* value_precursor_grad, void* value_from_first_cell_grad,
    void* learning_rate_lora_grad, void* weight_decay_lora_grad, void* value_residual_lora_grad,
    float* learning_rate_bias_grad, float* weight_decay_bias_grad,
    float* value_residual_bias_grad, float* key_replacement_grad, float* key_removal_grad,
    void* workspace, int64_t workspace_bytes, void* stream) {
  if (int rc = check_prepare(key_precursor, value_precursor, value_from_first_cell,
                             learning_rate_lora, weight_decay_lora, value_residual_lora,
                             learning_rate_bias, weight_decay_bias, value_residual_bias,
                             key_replacement, key_removal, rows, num_heads, head_size, dtype,
                             out_dtype))
    return rc;
  const bool res = value_residual_bias != nullptr;
  if (!learning_rate_bias_grad || !weight_decay_bias_grad || !key_replacement_grad ||
      !key_removal_grad || (res && !value_residual_bias_grad))
    return WKV7_ERR_NULL_POINTER;
  if (!res && (value_from_first_cell_grad || value_residual_lora_grad || value_residual_bias_grad))
    return WKV7_ERR_SHAPE;
  const void* grads_in[] = {weight_decay_grad, replacement_key_grad, value_grad,
                            removal_key_normalized_grad, replacement_grad};
  void* grads_out[] = {key_precursor_grad,    value_precursor_grad,   learning_rate_lora_grad,
                       weight_decay_lora_grad, value_from_first_cell_grad, value_residual_lora_grad};
  if (rows > 0) {
    for (const void* p : grads_in)
      if (!p) return WKV7_ERR_NULL_POINTER;
    for (int k = 0; k < (res ? 6 : 4); ++k)
      if (!grads_out[k]) return WKV7_ERR_NULL_POINTER;
  }
  const int64_t need = prepare_workspace(rows, num_heads);
  if (need > 0 && (!workspace || workspace_bytes < need)) return WKV7_ERR_SHAPE;
  for (const void* p : grads_in)
    if (p && !aligned_for(p, out_dtype)) return WKV7_ERR_ALIGNMENT;
  for (const void* p : grads_out)
    if (p && !aligned_for(p, dtype)) return WKV7_ERR_ALIGNMENT;
  float* sums[] = {learning_rate_bias_grad, weight_decay_bias_grad, key_replacement_grad,
                   key_removal_grad, value_residual_bias_grad};
  for (const float* p : sums)
    if (p && !aligned_for(p, WKV7_DTYPE_F32)) return WKV7_ERR_ALIGNMENT;
  if (workspace && !aligned_for(workspace, WKV7_DTYPE_F32)) return WKV7_ERR_ALIGNMENT;
  const int64_t C = num_heads * 64, in = rows * C * esize(dtype), out = rows * C * esize(out_dtype);
  std::vector<Range> o, i;
  for (void* p : grads_out) o.push_back({p, in});
  for (float* p : sums) o.push_back({p, C * 4});
  o.push_back({workspace, need});
  for (const void* p : {key_precursor, value_precursor, value_from_first_cell, learning_rate_lora,
                        weight_decay_lora, value_residual_lora})
    i.push_back({p, in});
  for (const float* p : {learning_rate_bias, weight_decay_bias, value_residual_bias,
                         key_replacement, key_removal})
    i.push_back({p, C * 4});
  for (const void* p : grads_in) i.push_back({p, out});
  if (any_overlap(o, i)) return WKV7_ERR_OVERLAP;
  rwkv_nb::PrepareArgs a = prepare_args(
      key_precursor, value_precursor, value_from_first_cell, learning_rate_lora,
      weight_decay_lora, value_residual_lora, learning_rate_bias, weight_decay_bias,
      value_residual_bias, key_replacement, key_removal, rows, num_heads, dtype, out_dtype);
  a.weight_decay_grad = weight_decay_grad;
  a.replacement_key_grad = replacement_key_grad;
  a.value_out_grad = value_grad;
  a.removal_grad = removal_key_normalized_grad;
  a.replacement_grad = replacement_grad;
  a.key_grad = key_precursor_grad;
  a.value_grad = value_precursor_grad;
  a.value_first_grad = value_from_first_cell_grad;
  a.lr_grad = learning_rate_lora_grad;
  a.wd_grad = weight_decay_lora_grad;
  a.vr_grad = value_residual_lora_grad;
  for (int k = 0; k < rwkv_nb::kPrepareSums; ++k) a.sums[k] = sums[k];
  a.workspace = static_cast<float*>(workspace);
  return wkv7::hip_status(rwkv_nb::launch_prepare_backward(a, static_cast<hipStream_t>(stream)));
}

}  // extern "C"
