// C ABI of the fused cross entropy + l2wrap (include/rwkv_lm_loss.h):
// argument validation on the host, before any HIP call, then dispatch.
#include "../../include/rwkv_lm_loss.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <initializer_list>

#include "lm_loss_launch.hpp"
#include "wkv7_launch.hpp"

namespace {

struct Span {
  const void* p;
  int64_t bytes;
};

bool overlaps(const Span& x, const Span& y) {
  if (!x.p || !y.p || x.bytes <= 0 || y.bytes <= 0) return false;
  const auto a0 = reinterpret_cast<uintptr_t>(x.p), b0 = reinterpret_cast<uintptr_t>(y.p);
  return a0 < b0 + static_cast<uintptr_t>(y.bytes) && b0 < a0 + static_cast<uintptr_t>(x.bytes);
}

// every output against every other output and every input
bool any_overlap(std::initializer_list<Span> outs, std::initializer_list<Span> ins) {
  for (auto i = outs.begin(); i != outs.end(); ++i) {
    for (auto j = i + 1; j != outs.end(); ++j)
      if (overlaps(*i, *j)) return true;
    for (const Span& in : ins)
      if (overlaps(*i, in)) return true;
  }
  return false;
}

bool aligned(const void* p, uintptr_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

// vector accesses when every row is a whole number of 8-logit pieces
uintptr_t row_alignment(int64_t vocab, int dtype) {
  if (vocab % rwkv_loss::kPiece == 0) return 16;
  return dtype == WKV7_DTYPE_BF16 ? 2 : 4;
}

int check_common(const void* logits, const int64_t* targets, int64_t rows, int64_t vocab,
                 int dtype) {
  if (dtype != WKV7_DTYPE_F32 && dtype != WKV7_DTYPE_BF16) return WKV7_ERR_DTYPE;
  if (rows < 0 || rows > INT32_MAX) return WKV7_ERR_SHAPE;   // one block per row
  if (vocab <= 0 || vocab > INT32_MAX) return WKV7_ERR_SHAPE;
  if (rows > 0 && vocab > INT64_MAX / 4 / rows) return WKV7_ERR_SHAPE;  // byte sizes fit int64
  if (rows > 0 && (!logits || !targets)) return WKV7_ERR_NULL_POINTER;
  if (!aligned(logits, row_alignment(vocab, dtype)) || !aligned(targets, 8))
    return WKV7_ERR_ALIGNMENT;
  return WKV7_OK;
}

}  // namespace

extern "C" {

int rwkv_cross_entropy_l2wrap_forward(const void* logits, const int64_t* targets, int64_t rows,
                                      int64_t vocab, int dtype, float* row_loss, float* row_lse,
                                      float* row_max, int32_t* row_argmax, void* stream) {
  if (int rc = check_common(logits, targets, rows, vocab, dtype)) return rc;
  if (rows > 0 && (!row_loss || !row_lse || !row_max || !row_argmax)) return WKV7_ERR_NULL_POINTER;
  for (const void* p : {static_cast<const void*>(row_loss), static_cast<const void*>(row_lse),
                        static_cast<const void*>(row_max), static_cast<const void*>(row_argmax)})
    if (!aligned(p, 4)) return WKV7_ERR_ALIGNMENT;
  const int64_t lb = rows * vocab * (dtype == WKV7_DTYPE_BF16 ? 2 : 4), rb = rows * 4;
  if (any_overlap({{row_loss, rb}, {row_lse, rb}, {row_max, rb}, {row_argmax, rb}},
                  {{logits, lb}, {targets, rows * 8}}))
    return WKV7_ERR_OVERLAP;
  rwkv_loss::XentArgs a{};
  a.logits = logits;
  a.targets = targets;
  a.rows = rows;
  a.vocab = vocab;
  a.bf16 = dtype == WKV7_DTYPE_BF16;
  a.row_loss = row_loss;
  a.row_lse = row_lse;
  a.row_max = row_max;
  a.row_argmax = row_argmax;
  return wkv7::hip_status(rwkv_loss::launch_xent_forward(a, static_cast<hipStream_t>(stream)));
}

int rwkv_cross_entropy_l2wrap_backward(const void* logits, const int64_t* targets,
                                       const float* row_lse, const float* row_max,
                                       const int32_t* row_argmax, const float* row_loss_grad,
                                       float l2wrap_scale, int64_t rows, int64_t vocab, int dtype,
                                       void* logits_grad, void* stream) {
  if (int rc = check_common(logits, targets, rows, vocab, dtype)) return rc;
  if (!(l2wrap_scale == l2wrap_scale) || l2wrap_scale == INFINITY || l2wrap_scale == -INFINITY)
    return WKV7_ERR_SHAPE;
  if (rows > 0 && (!row_lse || !row_max || !row_argmax || !row_loss_grad || !logits_grad))
    return WKV7_ERR_NULL_POINTER;
  for (const void* p : {static_cast<const void*>(row_lse), static_cast<const void*>(row_max),
                        static_cast<const void*>(row_argmax),
                        static_cast<const void*>(row_loss_grad)})
    if (!aligned(p, 4)) return WKV7_ERR_ALIGNMENT;
  if (!aligned(logits_grad, row_alignment(vocab, dtype))) return WKV7_ERR_ALIGNMENT;
  const int64_t lb = rows * vocab * (dtype == WKV7_DTYPE_BF16 ? 2 : 4), rb = rows * 4;
  if (any_overlap({{logits_grad, lb}},
                  {{logits, lb}, {targets, rows * 8}, {row_lse, rb}, {row_max, rb},
                   {row_argmax, rb}, {row_loss_grad, rb}}))
    return WKV7_ERR_OVERLAP;
  rwkv_loss::XentArgs a{};
  a.logits = logits;
  a.targets = targets;
  a.rows = rows;
  a.vocab = vocab;
  a.bf16 = dtype == WKV7_DTYPE_BF16;
  a.lse = row_lse;
  a.max = row_max;
  a.argmax = row_argmax;
  a.row_grad = row_loss_grad;
  a.l2wrap_scale = l2wrap_scale;
  a.logits_grad = logits_grad;
  return wkv7::hip_status(rwkv_loss::launch_xent_backward(a, static_cast<hipStream_t>(stream)));
}

}  // extern "C"
