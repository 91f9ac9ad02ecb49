// PyTorch-ROCm extension module `mask_loss`: the reference's operator surface
// (src/bindings.cpp:157-169, all-positional arguments) over the C ABI of
// libmask_loss_hip.so (include/mask_loss_hip.h).  Tensors are validated the
// way the reference validates them (device + contiguous, shapes, ranges),
// outputs and workspaces come from PyTorch's caching allocator, and every
// launch goes to the current HIP stream.  There is no CPU implementation:
// host tensors raise, as in the reference (src/cuda/utils.h:4-6,
// src/cpu/matching.cpp:618).
#include <ATen/hip/HIPContext.h>
#include <torch/csrc/autograd/custom_function.h>
#include <torch/extension.h>

#include <chrono>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/mask_loss_hip.h"

namespace {

#define ML_CHECK_INPUT(x)                                              \
  TORCH_CHECK((x).is_cuda(), #x " must be a CUDA tensor");             \
  TORCH_CHECK((x).is_contiguous(), #x " must be contiguous")

int dtype_code(const torch::Tensor& t, const char* name) {
  switch (t.scalar_type()) {
    case torch::kFloat32: return ML_F32;
    case torch::kBFloat16: return ML_BF16;
    case torch::kFloat16: return ML_F16;
    default: TORCH_CHECK(false, name, " must be float32, bfloat16 or float16");
  }
  return -1;
}

void ml_ok(int rc) { TORCH_CHECK(rc == ML_OK, ml_last_error()); }

ml_stream_t cur_stream() { return (ml_stream_t)at::hip::getCurrentHIPStream().stream(); }

// The forward's void-class check writes its answer into a pinned, coherent
// host word (mapped for the device) with a system-scope store; the host
// polls the word rather than recording an event in the stream (an event's
// system-scope release would stall the next kernel).  Words 4 .. 6 of the
// same block receive the column-tile classes' task counts, so that the
// forward launches only the classes that have images.  One block per host
// thread and device, kept for the life of the process.
struct VoidSlot {
  volatile int32_t* host = nullptr;
  int32_t* dev = nullptr;
};
constexpr int kClassWords = 4;  // offset of the class-count words in the block

VoidSlot& void_slot() {
  constexpr int kMaxDevices = 64;
  static thread_local VoidSlot slots[kMaxDevices];
  int dev = 0;
  TORCH_CHECK(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices,
              "no current HIP device");
  VoidSlot& v = slots[dev];
  if (!v.host) {
    void* h = nullptr;
    void* d = nullptr;
    TORCH_CHECK(hipHostMalloc(&h, 64, hipHostMallocMapped | hipHostMallocCoherent) == hipSuccess,
                "cannot allocate the pinned void-check word");
    TORCH_CHECK(hipHostGetDevicePointer(&d, h, 0) == hipSuccess, "cannot map the void-check word");
    v.dev = (int32_t*)d;
    v.host = (volatile int32_t*)h;
  }
  return v;
}

// Wait until the device has written the word (it holds -1 until then); if
// that takes unusually long, drain the stream, after which it is written.
int32_t wait_void_word(const VoidSlot& v, ml_stream_t stream) {
  const auto t0 = std::chrono::steady_clock::now();
  for (int32_t x = *v.host; x == -1; x = *v.host) {
    if (std::chrono::steady_clock::now() - t0 > std::chrono::seconds(2)) {
      TORCH_CHECK(hipStreamSynchronize((hipStream_t)stream) == hipSuccess, "void check: stream failed");
      const int32_t y = *v.host;
      TORCH_CHECK(y != -1, "void check: the flag was not written");
      return y;
    }
    std::this_thread::yield();
  }
  return *v.host;
}

torch::Tensor workspace(size_t bytes, const torch::Tensor& like) {
  return torch::empty({(int64_t)std::max<size_t>(bytes, 256)},
                      like.options().dtype(torch::kUInt8));
}

ml_shape make_shape(const torch::Tensor& mask_logits, const torch::Tensor& mask_targets,
                    const torch::Tensor& cls_logits, const torch::Tensor& cls_targets) {
  TORCH_CHECK(mask_logits.dim() == 5, "mask_logits must be (L,B,Q,H,W)");
  TORCH_CHECK(mask_targets.dim() == 3, "mask_targets must be (B,H_t,W_t)");
  TORCH_CHECK(cls_logits.dim() == 4, "cls_logits must be (L,B,Q,C)");
  TORCH_CHECK(cls_targets.dim() == 2, "cls_targets must be (B,GT)");
  TORCH_CHECK(mask_targets.scalar_type() == torch::kLong, "mask_targets must be int64");
  TORCH_CHECK(cls_targets.scalar_type() == torch::kLong, "cls_targets must be int64");
  ml_shape s;
  s.L = mask_logits.size(0);
  s.B = mask_logits.size(1);
  s.Q = mask_logits.size(2);
  s.H = mask_logits.size(3);
  s.W = mask_logits.size(4);
  s.Ht = mask_targets.size(1);
  s.Wt = mask_targets.size(2);
  s.C = cls_logits.size(3);
  s.GT_total = cls_targets.size(1);
  TORCH_CHECK(mask_targets.size(0) == s.B, "Batch size mismatch between logits and targets");
  TORCH_CHECK(cls_targets.size(0) == s.B, "Batch size mismatch between logits and cls targets");
  TORCH_CHECK(cls_logits.size(0) == s.L && cls_logits.size(1) == s.B && cls_logits.size(2) == s.Q,
              "cls_logits must match mask logits dimensions");
  const auto dev = mask_logits.device();
  TORCH_CHECK(mask_targets.device() == dev && cls_logits.device() == dev &&
                  cls_targets.device() == dev,
              "all tensors must be on the same device");
  return s;
}

ml_params make_params(double smooth, double sigmoid_scale, double dice_scale, double cls_scale,
                      int64_t background_index, double ug, double ug_min, double inf_thresh,
                      double num_masks, bool force_cls, bool force_masks, int64_t topk,
                      int64_t strategy, double mask_gamma, double mask_alpha, double cls_gamma,
                      double cls_alpha, int64_t void_idx, bool use_softmax, bool normalize) {
  ml_params p;
  p.smooth = (float)smooth;
  p.sigmoid_scale = (float)sigmoid_scale;
  p.dice_scale = (float)dice_scale;
  p.cls_scale = (float)cls_scale;
  p.background_index = background_index;
  p.uncertainty_gamma = (float)ug;
  p.uncertainty_gamma_min = (float)ug_min;
  p.inf_thresh = inf_thresh;
  p.num_masks = num_masks;
  p.force_unmatched_class_to_background = force_cls;
  p.force_unmatched_masks_to_empty = force_masks;
  p.topk_matches = topk;
  p.strategy_id = strategy;
  p.mask_gamma = (float)mask_gamma;
  p.mask_alpha = (float)mask_alpha;
  p.cls_gamma = (float)cls_gamma;
  p.cls_alpha = (float)cls_alpha;
  p.void_class_index = void_idx;
  p.use_softmax_label_loss = use_softmax;
  p.normalize_uncertainty = normalize;
  return p;
}

int64_t gt_out_of(int64_t GT_total, int64_t bg) {
  return GT_total - ((bg >= 0 && bg < GT_total) ? 1 : 0);
}

// --------------------------------------------------------------------------
// pairwise_mask_loss_forward  (src/bindings.cpp:164, src/cuda/pw_mask.cu:314)
// --------------------------------------------------------------------------
torch::Tensor pairwise_mask_loss_forward(const torch::Tensor& mask_logits,
                                         const torch::Tensor& mask_targets,
                                         const torch::Tensor& cls_logits,
                                         const torch::Tensor& cls_targets, double smooth,
                                         double sigmoid_scale, double dice_scale,
                                         double cls_scale, int64_t background_index, double ug,
                                         double ug_min, double mask_gamma, double mask_alpha,
                                         double cls_gamma, double cls_alpha, bool use_softmax,
                                         bool normalize) {
  ML_CHECK_INPUT(mask_logits);
  ML_CHECK_INPUT(mask_targets);
  ML_CHECK_INPUT(cls_logits);
  ML_CHECK_INPUT(cls_targets);
  const ml_shape s = make_shape(mask_logits, mask_targets, cls_logits, cls_targets);
  const ml_params p = make_params(smooth, sigmoid_scale, dice_scale, cls_scale, background_index,
                                  ug, ug_min, 1e30, -1.0, false, false, 1, 0, mask_gamma,
                                  mask_alpha, cls_gamma, cls_alpha, -1, use_softmax, normalize);
  const int64_t GT_out = gt_out_of(s.GT_total, background_index);
  const int mdt = dtype_code(mask_logits, "mask_logits");
  const int cdt = dtype_code(cls_logits, "cls_logits");
  if (GT_out == 0)  // reference returns (L,B,Q,0) here (pw_mask.cu:402-404)
    return torch::zeros({s.L, s.B, s.Q, 0}, mask_logits.options().dtype(torch::kFloat32));
  auto out = torch::empty({3, s.L, s.B, s.Q, GT_out}, mask_logits.options().dtype(torch::kFloat32));
  const size_t wsb = ml_pairwise_mask_loss_workspace_size(&s, &p, mdt);
  TORCH_CHECK(wsb > 0 || s.B == 0, "unsupported shape");
  auto ws = workspace(wsb, mask_logits);
  ml_ok(ml_pairwise_mask_loss_forward(&s, &p, mdt, mask_logits.data_ptr(),
                                      mask_targets.data_ptr<int64_t>(), cdt, cls_logits.data_ptr(),
                                      cls_targets.data_ptr<int64_t>(), out.data_ptr<float>(),
                                      ws.data_ptr(), ws.numel(), cur_stream()));
  return out;
}

// --------------------------------------------------------------------------
// mask_matching  (src/bindings.cpp:165, src/cpu/matching.cpp:592)
// --------------------------------------------------------------------------
std::vector<torch::Tensor> matching_impl(const torch::Tensor& mask_logits,
                                         const torch::Tensor& mask_targets,
                                         const torch::Tensor& cls_logits,
                                         const torch::Tensor& cls_targets, const ml_params& p,
                                         bool want_saved,
                                         const c10::optional<torch::Tensor>& grad_prefill,
                                         bool check_void = false) {
  ML_CHECK_INPUT(mask_logits);
  ML_CHECK_INPUT(mask_targets);
  ML_CHECK_INPUT(cls_logits);
  ML_CHECK_INPUT(cls_targets);
  const ml_shape s = make_shape(mask_logits, mask_targets, cls_logits, cls_targets);
  const int mdt = dtype_code(mask_logits, "mask_logits");
  const int cdt = dtype_code(cls_logits, "cls_logits");
  auto i64 = mask_logits.options().dtype(torch::kLong);
  auto f32 = mask_logits.options().dtype(torch::kFloat32);
  auto pred_to_gt = torch::empty({s.L, s.B, s.Q}, i64);
  auto pred_round = torch::empty({s.L, s.B, s.Q}, i64);
  auto means = torch::empty({3, s.L}, f32);
  torch::Tensor saved;
  if (want_saved)
    saved = torch::empty({(int64_t)std::max<size_t>(ml_saved_bytes(&s, &p, mdt), 256)},
                         mask_logits.options().dtype(torch::kUInt8));
  void* prefill = nullptr;
  if (grad_prefill.has_value()) {
    const auto& g = *grad_prefill;
    ML_CHECK_INPUT(g);
    TORCH_CHECK(want_saved, "grad_prefill needs the fused forward");
    TORCH_CHECK(g.sizes() == mask_logits.sizes() && g.scalar_type() == mask_logits.scalar_type() &&
                    g.device() == mask_logits.device(),
                "grad_prefill must match mask_logits in shape, dtype and device");
    prefill = g.data_ptr();
  }
  const size_t wsb = ml_mask_matching_workspace_size(&s, &p, mdt);
  TORCH_CHECK(wsb > 0 || s.B == 0 || s.L == 0, ml_last_error());
  auto ws = workspace(wsb, mask_logits);
  VoidSlot& words = void_slot();
  VoidSlot* vs = check_void ? &words : nullptr;
  if (vs) *vs->host = -1;
  const int rc = ml_mask_matching_forward_polled(
      &s, &p, mdt, mask_logits.data_ptr(), mask_targets.data_ptr<int64_t>(), cdt,
      cls_logits.data_ptr(), cls_targets.data_ptr<int64_t>(), pred_to_gt.data_ptr<int64_t>(),
      pred_round.data_ptr<int64_t>(), means.data_ptr<float>(), nullptr,
      want_saved ? saved.data_ptr() : nullptr, prefill, vs ? vs->dev : nullptr,
      nullptr, ws.data_ptr(), ws.numel(), cur_stream(), words.dev + kClassWords,
      words.host + kClassWords);
  if (rc != ML_OK) {
    // a failure after the first launch leaves kernels queued that may still
    // write this thread's void and class-count words: let them finish before
    // the next call re-arms them
    const std::string msg = ml_last_error();
    (void)hipStreamSynchronize((hipStream_t)cur_stream());
    TORCH_CHECK(false, msg);
  }
  int32_t void_hit = -1;
  if (vs) void_hit = wait_void_word(*vs, cur_stream());  // the rest of the forward stays queued
  // means follow the logits dtype (src/cuda/mask_matching_forward.cu:580-583);
  // the fused entry keeps them in float32
  const auto out_dt = want_saved ? torch::kFloat32 : mask_logits.scalar_type();
  std::vector<torch::Tensor> r = {pred_to_gt, pred_round, means[0].to(out_dt),
                                  means[1].to(out_dt), means[2].to(out_dt)};
  if (want_saved) r.push_back(saved);
  if (check_void) r.push_back(torch::full({1}, void_hit, torch::dtype(torch::kInt32)));
  return r;
}

std::vector<torch::Tensor> mask_matching(
    const torch::Tensor& mask_logits, const torch::Tensor& mask_targets,
    const torch::Tensor& cls_logits, const torch::Tensor& cls_targets, double smooth,
    double sigmoid_scale, double dice_scale, double cls_scale, int64_t background_index, double ug,
    double ug_min, double inf_thresh, double num_masks, bool force_cls, bool force_masks,
    int64_t topk, int64_t strategy, double mask_gamma, double mask_alpha, double cls_gamma,
    double cls_alpha, int64_t void_idx, bool use_softmax, bool normalize) {
  const ml_params p = make_params(smooth, sigmoid_scale, dice_scale, cls_scale, background_index,
                                  ug, ug_min, inf_thresh, num_masks, force_cls, force_masks, topk,
                                  strategy, mask_gamma, mask_alpha, cls_gamma, cls_alpha, void_idx,
                                  use_softmax, normalize);
  return matching_impl(mask_logits, mask_targets, cls_logits, cls_targets, p, false,
                       c10::nullopt);
}

// The reference's MaskMatchingFunction passes normalize_uncertainty a second
// time after uncertainty_gamma_min (functions/mask/matching.py:198-224); this
// overload accepts that 25-argument call.
std::vector<torch::Tensor> mask_matching_wrapper_order(
    const torch::Tensor& mask_logits, const torch::Tensor& mask_targets,
    const torch::Tensor& cls_logits, const torch::Tensor& cls_targets, double smooth,
    double sigmoid_scale, double dice_scale, double cls_scale, int64_t background_index, double ug,
    double ug_min, bool normalize_early, double inf_thresh, double num_masks, bool force_cls,
    bool force_masks, int64_t topk, int64_t strategy, double mask_gamma, double mask_alpha,
    double cls_gamma, double cls_alpha, int64_t void_idx, bool use_softmax, bool normalize) {
  (void)normalize_early;
  return mask_matching(mask_logits, mask_targets, cls_logits, cls_targets, smooth, sigmoid_scale,
                       dice_scale, cls_scale, background_index, ug, ug_min, inf_thresh, num_masks,
                       force_cls, force_masks, topk, strategy, mask_gamma, mask_alpha, cls_gamma,
                       cls_alpha, void_idx, use_softmax, normalize);
}

// Same as mask_matching, plus a sixth output: the saved state (per-query
// statistics, matched rows, compact labels) the fused backward uses to read
// every matched logit once.  With grad_prefill (the tensor that will receive
// the mask-logit gradient) the forward zero-fills it beside the assignment.
// With check_void, a seventh output (CPU int32, one element) says whether
// cls_targets holds void_class_index (1), not (0), or no valid index was
// given (0); the call then waits for the forward's preparation kernels.
std::vector<torch::Tensor> mask_matching_fused(
    const torch::Tensor& mask_logits, const torch::Tensor& mask_targets,
    const torch::Tensor& cls_logits, const torch::Tensor& cls_targets, double smooth,
    double sigmoid_scale, double dice_scale, double cls_scale, int64_t background_index, double ug,
    double ug_min, double inf_thresh, double num_masks, bool force_cls, bool force_masks,
    int64_t topk, int64_t strategy, double mask_gamma, double mask_alpha, double cls_gamma,
    double cls_alpha, int64_t void_idx, bool use_softmax, bool normalize,
    const c10::optional<torch::Tensor>& grad_prefill, bool check_void) {
  const ml_params p = make_params(smooth, sigmoid_scale, dice_scale, cls_scale, background_index,
                                  ug, ug_min, inf_thresh, num_masks, force_cls, force_masks, topk,
                                  strategy, mask_gamma, mask_alpha, cls_gamma, cls_alpha, void_idx,
                                  use_softmax, normalize);
  return matching_impl(mask_logits, mask_targets, cls_logits, cls_targets, p, true, grad_prefill,
                       check_void);
}

// --------------------------------------------------------------------------
// mask_matching_backward  (src/bindings.cpp:166, mask_matching_backward.cu:378)
// --------------------------------------------------------------------------
std::vector<torch::Tensor> backward_impl(
    const torch::Tensor& g_mask, const torch::Tensor& g_dice, const torch::Tensor& g_cls,
    const torch::Tensor& mask_logits, const torch::Tensor& mask_targets,
    const torch::Tensor& cls_logits, const torch::Tensor& cls_targets,
    const torch::Tensor& pred_to_gt, const ml_params& p, const torch::Tensor* saved,
    const c10::optional<torch::Tensor>& grad_prefill) {
  ML_CHECK_INPUT(mask_logits);
  ML_CHECK_INPUT(mask_targets);
  ML_CHECK_INPUT(cls_logits);
  ML_CHECK_INPUT(cls_targets);
  ML_CHECK_INPUT(pred_to_gt);
  const ml_shape s = make_shape(mask_logits, mask_targets, cls_logits, cls_targets);
  TORCH_CHECK(pred_to_gt.scalar_type() == torch::kLong, "pred_to_gt must be int64");
  TORCH_CHECK(pred_to_gt.dim() == 3 && pred_to_gt.size(0) == s.L && pred_to_gt.size(1) == s.B &&
                  pred_to_gt.size(2) == s.Q,
              "pred_to_gt must have shape (L,B,Q)");
  auto f32 = mask_logits.options().dtype(torch::kFloat32);
  auto gm = g_mask.to(f32).contiguous();
  auto gd = g_dice.to(f32).contiguous();
  auto gc = g_cls.to(f32).contiguous();
  TORCH_CHECK(gm.numel() == s.L && gd.numel() == s.L && gc.numel() == s.L,
              "upstream gradients must have shape (L,)");
  const int mdt = dtype_code(mask_logits, "mask_logits");
  const int cdt = dtype_code(cls_logits, "cls_logits");
  torch::Tensor grad_mask;
  if (grad_prefill.has_value()) {
    TORCH_CHECK(saved != nullptr, "grad_prefill needs the saved state");
    grad_mask = *grad_prefill;
    ML_CHECK_INPUT(grad_mask);
    TORCH_CHECK(grad_mask.sizes() == mask_logits.sizes() &&
                    grad_mask.scalar_type() == mask_logits.scalar_type(),
                "grad_prefill must match mask_logits in shape and dtype");
  } else {
    grad_mask = torch::empty_like(mask_logits);
  }
  auto grad_cls = torch::empty_like(cls_logits);
  if (saved) {
    ML_CHECK_INPUT(*saved);
    TORCH_CHECK(saved->numel() >= (int64_t)ml_saved_bytes(&s, &p, mdt), "saved state size mismatch");
  }
  const size_t wsb = ml_mask_matching_backward_workspace_size(&s, &p, mdt);
  auto ws = workspace(wsb, mask_logits);
  ml_ok(ml_mask_matching_backward(
      &s, &p, gm.data_ptr<float>(), gd.data_ptr<float>(), gc.data_ptr<float>(), mdt,
      mask_logits.data_ptr(), mask_targets.data_ptr<int64_t>(), cdt, cls_logits.data_ptr(),
      cls_targets.data_ptr<int64_t>(), pred_to_gt.data_ptr<int64_t>(),
      saved ? saved->data_ptr() : nullptr, grad_prefill.has_value() ? 1 : 0, grad_mask.data_ptr(),
      grad_cls.data_ptr(), ws.data_ptr(), ws.numel(), cur_stream()));
  return {grad_mask, grad_cls};
}

std::vector<torch::Tensor> mask_matching_backward(
    const torch::Tensor& g_mask, const torch::Tensor& g_dice, const torch::Tensor& g_cls,
    const torch::Tensor& mask_logits, const torch::Tensor& mask_targets,
    const torch::Tensor& cls_logits, const torch::Tensor& cls_targets,
    const torch::Tensor& pred_to_gt, double smooth, double sigmoid_scale, double dice_scale,
    double cls_scale, int64_t background_index, double ug, double ug_min, double num_masks,
    bool force_cls, bool force_masks, double mask_gamma, double mask_alpha, double cls_gamma,
    double cls_alpha, int64_t void_idx, bool use_softmax, bool normalize) {
  const ml_params p = make_params(smooth, sigmoid_scale, dice_scale, cls_scale, background_index,
                                  ug, ug_min, 1e30, num_masks, force_cls, force_masks, 1, 0,
                                  mask_gamma, mask_alpha, cls_gamma, cls_alpha, void_idx,
                                  use_softmax, normalize);
  return backward_impl(g_mask, g_dice, g_cls, mask_logits, mask_targets, cls_logits, cls_targets,
                       pred_to_gt, p, nullptr, c10::nullopt);
}

std::vector<torch::Tensor> mask_matching_backward_fused(
    const torch::Tensor& g_mask, const torch::Tensor& g_dice, const torch::Tensor& g_cls,
    const torch::Tensor& mask_logits, const torch::Tensor& mask_targets,
    const torch::Tensor& cls_logits, const torch::Tensor& cls_targets,
    const torch::Tensor& pred_to_gt, double smooth, double sigmoid_scale, double dice_scale,
    double cls_scale, int64_t background_index, double ug, double ug_min, double num_masks,
    bool force_cls, bool force_masks, double mask_gamma, double mask_alpha, double cls_gamma,
    double cls_alpha, int64_t void_idx, bool use_softmax, bool normalize,
    const torch::Tensor& saved, const c10::optional<torch::Tensor>& grad_prefill) {
  const ml_params p = make_params(smooth, sigmoid_scale, dice_scale, cls_scale, background_index,
                                  ug, ug_min, 1e30, num_masks, force_cls, force_masks, 1, 0,
                                  mask_gamma, mask_alpha, cls_gamma, cls_alpha, void_idx,
                                  use_softmax, normalize);
  return backward_impl(g_mask, g_dice, g_cls, mask_logits, mask_targets, cls_logits, cls_targets,
                       pred_to_gt, p, &saved, grad_prefill);
}

// --------------------------------------------------------------------------
// MaskMatchingFunction's autograd node (reference functions/mask/matching.py:
// 33-334) in C++: the forward is mask_matching_fused with the gradient buffer
// prefilled and the void-class check, the backward mask_matching_backward_fused
// on the saved state.  The Python class keeps the reference's argument
// defaulting and validation and calls mask_matching_autograd; the node itself
// keeps the per-step host work to the launches (no Python frames in either
// direction).
// --------------------------------------------------------------------------
struct MatchingNode : public torch::autograd::Function<MatchingNode> {
  static torch::autograd::variable_list forward(torch::autograd::AutogradContext* ctx,
                                                const torch::Tensor& mask_logits,
                                                const torch::Tensor& mask_targets,
                                                const torch::Tensor& cls_logits,
                                                const torch::Tensor& cls_targets,
                                                const ml_params& p, bool check_void,
                                                bool want_prefill) {
    const auto z = mask_logits.contiguous();
    const auto t = mask_targets.contiguous();
    const auto zc = cls_logits.contiguous();
    const auto ct = cls_targets.contiguous();
    c10::optional<torch::Tensor> prefill;
    if (want_prefill) prefill = torch::empty_like(z, at::MemoryFormat::Contiguous);
    auto outs = matching_impl(z, t, zc, ct, p, true, prefill, check_void);
    // outs: pred_to_gt, pred_round, the three layer means, saved state[, void flag]
    ctx->save_for_backward({z, t, zc, ct, outs[0], outs[5]});
    // the parameters travel as the bytes of their C struct
    auto pb = torch::empty({(int64_t)sizeof(ml_params)}, torch::dtype(torch::kUInt8));
    std::memcpy(pb.data_ptr(), &p, sizeof(ml_params));
    ctx->saved_data["params"] = pb;
    // the zero-filled gradient buffer serves the first backward only (a
    // second backward through a retained graph gets a fresh tensor)
    if (prefill.has_value()) ctx->saved_data["prefill"] = *prefill;
    if (check_void && outs[6].item<int32_t>() == 1)
      TORCH_CHECK_VALUE(false, "cls_targets must not contain the void class index");
    ctx->mark_non_differentiable({outs[0], outs[1]});
    ctx->set_materialize_grads(false);  // no zero gradients for the integer outputs
    return {outs[0], outs[1], outs[2], outs[3], outs[4]};
  }

  static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                 torch::autograd::variable_list g) {
    const auto sv = ctx->get_saved_variables();
    const auto& z = sv[0];
    ml_params p;
    std::memcpy(&p, ctx->saved_data["params"].toTensor().data_ptr(), sizeof(ml_params));
    // as mask_matching_backward_fused: the assignment's own fields do not apply
    p.inf_thresh = 1e30;
    p.topk_matches = 1;
    p.strategy_id = 0;
    c10::optional<torch::Tensor> prefill;
    auto it = ctx->saved_data.find("prefill");
    if (it != ctx->saved_data.end()) {
      prefill = it->second.toTensor();
      ctx->saved_data.erase(it);
    }
    auto grad_of = [&](const torch::Tensor& x) {
      return x.defined() ? x.detach() : torch::zeros({z.size(0)}, z.options().dtype(torch::kFloat32));
    };
    const auto r = backward_impl(grad_of(g[2]), grad_of(g[3]), grad_of(g[4]), z, sv[1], sv[2],
                                 sv[3], sv[4], p, &sv[5], prefill);
    return {r[0], torch::Tensor(), r[1], torch::Tensor(), torch::Tensor(), torch::Tensor(),
            torch::Tensor()};
  }
};

std::vector<torch::Tensor> mask_matching_autograd(
    const torch::Tensor& mask_logits, const torch::Tensor& mask_targets,
    const torch::Tensor& cls_logits, const torch::Tensor& cls_targets, double smooth,
    double sigmoid_scale, double dice_scale, double cls_scale, int64_t background_index, double ug,
    double ug_min, double inf_thresh, double num_masks, bool force_cls, bool force_masks,
    int64_t topk, int64_t strategy, double mask_gamma, double mask_alpha, double cls_gamma,
    double cls_alpha, int64_t void_idx, bool use_softmax, bool normalize, bool check_void) {
  const ml_params p = make_params(smooth, sigmoid_scale, dice_scale, cls_scale, background_index,
                                  ug, ug_min, inf_thresh, num_masks, force_cls, force_masks, topk,
                                  strategy, mask_gamma, mask_alpha, cls_gamma, cls_alpha, void_idx,
                                  use_softmax, normalize);
  const bool want_prefill =
      torch::GradMode::is_enabled() && mask_logits.requires_grad() && !force_masks;
  return MatchingNode::apply(mask_logits, mask_targets, cls_logits, cls_targets, p, check_void,
                             want_prefill);
}

// --------------------------------------------------------------------------
// pairwise label losses (src/bindings.cpp:167-168)
// --------------------------------------------------------------------------
torch::Tensor label_impl(const torch::Tensor& logits, const torch::Tensor& targets,
                         int64_t background_index, double scale, double gamma, double alpha,
                         bool use_softmax) {
  ML_CHECK_INPUT(logits);
  ML_CHECK_INPUT(targets);
  TORCH_CHECK(logits.dim() == 4, "logits must be (L,B,Q,C)");
  TORCH_CHECK(targets.dim() == 2, "targets must be (B,GT)");
  TORCH_CHECK(targets.scalar_type() == torch::kLong, "targets must be int64");
  TORCH_CHECK(logits.size(1) == targets.size(0), "batch size mismatch between logits and targets");
  const int64_t L = logits.size(0), B = logits.size(1), Q = logits.size(2), C = logits.size(3);
  const int64_t GT_total = targets.size(1);
  const int64_t GT_out = gt_out_of(GT_total, background_index);
  auto out = torch::empty({L, B, Q, GT_out}, logits.options().dtype(torch::kFloat32));
  if (GT_out == 0) return out;
  ml_ok(ml_pairwise_label_loss_forward(L, B, Q, C, GT_total, dtype_code(logits, "logits"),
                                       logits.data_ptr(), targets.data_ptr<int64_t>(),
                                       background_index, (float)scale, (float)gamma, (float)alpha,
                                       use_softmax, out.data_ptr<float>(), cur_stream()));
  return out;
}

torch::Tensor forward_pw_sigmoid_label_loss(const torch::Tensor& logits,
                                            const torch::Tensor& targets,
                                            int64_t background_index, double scale, double gamma,
                                            double alpha) {
  return label_impl(logits, targets, background_index, scale, gamma, alpha, false);
}

torch::Tensor forward_pw_softmax_label_loss(const torch::Tensor& logits,
                                            const torch::Tensor& targets,
                                            int64_t background_index, double scale) {
  return label_impl(logits, targets, background_index, scale, 0.0, -1.0, true);
}

// --------------------------------------------------------------------------
// point-sampling front end (functions/utils.py:12-20, the *_sampling_py
// costs of functions/sigmoid/pw_sigmoid_ce.py:407-550 and
// functions/dice/pw_dice_loss.py:174-268 for given points)
// --------------------------------------------------------------------------
void check_coords(const torch::Tensor& coords, const torch::Tensor& like) {
  ML_CHECK_INPUT(coords);
  TORCH_CHECK(coords.scalar_type() == torch::kFloat32, "point coordinates must be float32");
  TORCH_CHECK(coords.size(-1) == 2, "point coordinates must end in a dimension of size 2 (x, y)");
  TORCH_CHECK(coords.device() == like.device(), "all tensors must be on the same device");
}

// (N, C, H, W) planes at (N, P, 2) or (N, Hg, Wg, 2) points -> (N, C, P) or (N, C, Hg, Wg)
torch::Tensor point_sample(const torch::Tensor& input, const torch::Tensor& coords,
                           bool align_corners) {
  ML_CHECK_INPUT(input);
  check_coords(coords, input);
  TORCH_CHECK(input.dim() == 4, "point_sample: input must be (N,C,H,W)");
  TORCH_CHECK(coords.dim() == 3 || coords.dim() == 4, "point_sample: coords must be (N,P,2) or (N,Hg,Wg,2)");
  TORCH_CHECK(coords.size(0) == input.size(0), "point_sample: batch size mismatch between input and coords");
  const int64_t N = input.size(0), C = input.size(1), H = input.size(2), W = input.size(3);
  const int64_t P = coords.dim() == 3 ? coords.size(1) : coords.size(1) * coords.size(2);
  TORCH_CHECK(H > 0 && W > 0, "point_sample: input must have positive spatial size");
  auto out = torch::empty({N, C, P}, input.options());
  ml_ok(ml_point_sample(dtype_code(input, "input"), input.data_ptr(), coords.data_ptr<float>(), N, C,
                        H, W, P, std::max<int64_t>(N, 1), align_corners ? 1 : 0, out.data_ptr(),
                        cur_stream()));
  if (coords.dim() == 4) return out.view({N, C, coords.size(1), coords.size(2)});
  return out;
}

// gradient of point_sample with respect to its (N, C, H, W) input
torch::Tensor point_sample_backward(const torch::Tensor& grad_out, const torch::Tensor& coords,
                                    int64_t H, int64_t W, bool align_corners) {
  ML_CHECK_INPUT(grad_out);
  check_coords(coords, grad_out);
  TORCH_CHECK(grad_out.dim() == 3 || grad_out.dim() == 4, "point_sample backward: grad must be (N,C,P) or (N,C,Hg,Wg)");
  TORCH_CHECK(coords.dim() == grad_out.dim() && coords.size(0) == grad_out.size(0),
              "point_sample backward: coords do not match the gradient");
  const int64_t N = grad_out.size(0), C = grad_out.size(1);
  const int64_t P = grad_out.dim() == 3 ? grad_out.size(2) : grad_out.size(2) * grad_out.size(3);
  const int64_t Pc = coords.dim() == 3 ? coords.size(1) : coords.size(1) * coords.size(2);
  TORCH_CHECK(P == Pc, "point_sample backward: coords do not match the gradient");
  TORCH_CHECK(H > 0 && W > 0, "point_sample backward: input must have positive spatial size");
  const int dt = dtype_code(grad_out, "grad");
  auto gin = torch::empty({N, C, H, W}, grad_out.options());
  const size_t wsb = ml_point_sample_backward_workspace_size(dt, N, C, H, W, P, std::max<int64_t>(N, 1));
  auto ws = workspace(wsb, grad_out);
  ml_ok(ml_point_sample_backward(dt, grad_out.data_ptr(), coords.data_ptr<float>(), N, C, H, W, P,
                                 std::max<int64_t>(N, 1), align_corners ? 1 : 0, gin.data_ptr(),
                                 wsb ? (float*)ws.data_ptr() : nullptr, wsb, cur_stream()));
  return gin;
}

// (L, B, Q, H, W) logits at one (B, P, 2) point set per image -> (L, B, Q, P)
torch::Tensor point_sample_masks(const torch::Tensor& logits, const torch::Tensor& coords,
                                 bool align_corners) {
  ML_CHECK_INPUT(logits);
  check_coords(coords, logits);
  TORCH_CHECK(logits.dim() == 5, "logits must be (L,B,Q,H,W)");
  TORCH_CHECK(coords.dim() == 3 && coords.size(0) == logits.size(1),
              "point coordinates must be (B,P,2) with the logits' batch size");
  const int64_t L = logits.size(0), B = logits.size(1), Q = logits.size(2);
  const int64_t H = logits.size(3), W = logits.size(4), P = coords.size(1);
  TORCH_CHECK(H > 0 && W > 0, "mask_logits must have positive spatial size");
  auto out = torch::empty({L, B, Q, P}, logits.options());
  ml_ok(ml_point_sample(dtype_code(logits, "logits"), logits.data_ptr(), coords.data_ptr<float>(),
                        L * B, Q, H, W, P, std::max<int64_t>(B, 1), align_corners ? 1 : 0,
                        out.data_ptr(), cur_stream()));
  return out;
}

torch::Tensor point_labels(const torch::Tensor& targets, const torch::Tensor& coords) {
  ML_CHECK_INPUT(targets);
  check_coords(coords, targets);
  TORCH_CHECK(targets.dim() == 3, "targets must be (B,H_t,W_t)");
  TORCH_CHECK(targets.scalar_type() == torch::kLong, "targets must be int64");
  TORCH_CHECK(coords.dim() == 3 && coords.size(0) == targets.size(0),
              "point coordinates must be (B,P,2) with the targets' batch size");
  const int64_t B = targets.size(0), P = coords.size(1);
  TORCH_CHECK(targets.size(1) > 0 && targets.size(2) > 0, "targets must have positive spatial size");
  auto out = torch::empty({B, P}, targets.options());
  ml_ok(ml_point_labels(targets.data_ptr<int64_t>(), coords.data_ptr<float>(), B, targets.size(1),
                        targets.size(2), P, out.data_ptr<int64_t>(), cur_stream()));
  return out;
}

// GT_total = max of the full label map + 1, read back to the host as the
// reference does (pw_sigmoid_ce.py:466-467, pw_dice_loss.py:209-210).
torch::Tensor pairwise_points_impl(const torch::Tensor& logits, const torch::Tensor& targets,
                                   const torch::Tensor& coords, const ml_params& p, bool dice,
                                   bool align_corners) {
  ML_CHECK_INPUT(logits);
  ML_CHECK_INPUT(targets);
  check_coords(coords, logits);
  TORCH_CHECK(logits.dim() == 5, "logits must be (L,B,C,H,W)");
  TORCH_CHECK(targets.dim() == 3, "targets must be (B,H_t,W_t)");
  TORCH_CHECK(targets.scalar_type() == torch::kLong, "targets must be int64");
  TORCH_CHECK(targets.size(0) == logits.size(1), "Batch size mismatch between logits and targets");
  TORCH_CHECK(targets.device() == logits.device(), "all tensors must be on the same device");
  TORCH_CHECK(coords.dim() == 3 && coords.size(0) == logits.size(1),
              "point coordinates must be (B,P,2) with the logits' batch size");
  TORCH_CHECK(coords.size(1) > 0, "num_points must be > 0");
  TORCH_CHECK(targets.size(1) > 0 && targets.size(2) > 0, "targets must have positive spatial size");
  const int64_t gt_total =
      targets.numel() > 0 ? std::max<int64_t>(targets.max().item<int64_t>() + 1, 0) : 0;
  const int64_t L = logits.size(0), B = logits.size(1), C = logits.size(2), P = coords.size(1);
  auto f32 = logits.options().dtype(torch::kFloat32);
  const int64_t GT_out = gt_out_of(gt_total, p.background_index);
  if (GT_out == 0) return torch::zeros({L, B, C, 0}, f32);
  auto pts = point_sample_masks(logits, coords, align_corners);  // (L, B, C, P)
  ml_shape s;
  s.L = L;
  s.B = B;
  s.Q = C;
  s.H = 1;
  s.W = P;
  s.Ht = 1;
  s.Wt = P;
  s.C = 0;
  s.GT_total = gt_total;
  auto out = torch::empty({L, B, C, GT_out}, f32);
  const int dt = dtype_code(logits, "logits");
  const size_t wsb = ml_pairwise_points_workspace_size(&s, &p, dt, targets.size(1), targets.size(2));
  TORCH_CHECK(wsb > 0 || B == 0, ml_last_error());
  auto ws = workspace(wsb, logits);
  ml_ok(ml_pairwise_sigmoid_dice_points_forward(
      &s, &p, dt, pts.data_ptr(), targets.data_ptr<int64_t>(), targets.size(1), targets.size(2),
      coords.data_ptr<float>(), dice ? nullptr : out.data_ptr<float>(),
      dice ? out.data_ptr<float>() : nullptr, ws.data_ptr(), ws.numel(), cur_stream()));
  return out;
}

// focal BCE over the points, mean over the points (no uncertainty weights)
torch::Tensor forward_pw_sigmoid_ce_loss_sampling(const torch::Tensor& logits,
                                                  const torch::Tensor& targets,
                                                  const torch::Tensor& coords,
                                                  int64_t background_index, double scale,
                                                  double gamma, double alpha, bool align_corners) {
  ml_params p = make_params(1.0, scale, 1.0, 1.0, background_index, 0.0, 0.0, 1e30, -1.0, false,
                            false, 1, 0, gamma, alpha, 0.0, -1.0, -1, false, false);
  return pairwise_points_impl(logits, targets, coords, p, false, align_corners);
}

torch::Tensor forward_pw_dice_loss_sampling(const torch::Tensor& logits, const torch::Tensor& targets,
                                            const torch::Tensor& coords, double smooth,
                                            int64_t background_index, double scale,
                                            bool align_corners) {
  ml_params p = make_params(smooth, 1.0, scale, 1.0, background_index, 0.0, 0.0, 1e30, -1.0, false,
                            false, 1, 0, 0.0, -1.0, 0.0, -1.0, -1, false, false);
  return pairwise_points_impl(logits, targets, coords, p, true, align_corners);
}

// --------------------------------------------------------------------------
// standalone pairwise sigmoid CE / dice  (src/bindings.cpp:159,162)
// --------------------------------------------------------------------------
// GT_total = targets.max() + 1, read back to the host as the reference does
// (src/cuda/pw_sigmoid_ce.cu:222-224, src/cuda/pw_dice_loss.cu:132-134).
torch::Tensor pairwise_bd_impl(const torch::Tensor& logits, const torch::Tensor& targets,
                               const ml_params& p, bool dice) {
  ML_CHECK_INPUT(logits);
  ML_CHECK_INPUT(targets);
  TORCH_CHECK(logits.dim() == 5, "logits must be (L,B,C,H,W)");
  TORCH_CHECK(targets.dim() == 3, "targets must be (B,H_t,W_t)");
  TORCH_CHECK(targets.scalar_type() == torch::kLong, "targets must be int64");
  TORCH_CHECK(targets.size(0) == logits.size(1), "Batch size mismatch between logits and targets");
  TORCH_CHECK(targets.device() == logits.device(), "all tensors must be on the same device");
  const int64_t gt_total =
      targets.numel() > 0 ? std::max<int64_t>(targets.max().item<int64_t>() + 1, 0) : 0;
  ml_shape s;
  s.L = logits.size(0);
  s.B = logits.size(1);
  s.Q = logits.size(2);
  s.H = logits.size(3);
  s.W = logits.size(4);
  s.Ht = targets.size(1);
  s.Wt = targets.size(2);
  s.C = 0;
  s.GT_total = gt_total;
  const int64_t GT_out = gt_out_of(gt_total, p.background_index);
  auto f32 = logits.options().dtype(torch::kFloat32);
  if (GT_out == 0) return torch::zeros({s.L, s.B, s.Q, 0}, f32);
  auto out = torch::empty({s.L, s.B, s.Q, GT_out}, f32);
  const int dt = dtype_code(logits, "logits");
  const size_t wsb = ml_pairwise_mask_loss_workspace_size(&s, &p, dt);
  TORCH_CHECK(wsb > 0 || s.B == 0, ml_last_error());
  auto ws = workspace(wsb, logits);
  ml_ok(ml_pairwise_sigmoid_dice_forward(&s, &p, dt, logits.data_ptr(),
                                         targets.data_ptr<int64_t>(),
                                         dice ? nullptr : out.data_ptr<float>(),
                                         dice ? out.data_ptr<float>() : nullptr, ws.data_ptr(),
                                         ws.numel(), cur_stream()));
  return out;
}

torch::Tensor forward_pw_sigmoid_ce_loss(const torch::Tensor& logits, const torch::Tensor& targets,
                                         int64_t background_index, double scale, double gamma,
                                         double alpha, double ug, double ug_min, bool normalize) {
  ml_params p = make_params(1.0, scale, 1.0, 1.0, background_index, ug, ug_min, 1e30, -1.0, false,
                            false, 1, 0, gamma, alpha, 0.0, -1.0, -1, false, normalize);
  return pairwise_bd_impl(logits, targets, p, false);
}

torch::Tensor forward_pw_dice_loss(const torch::Tensor& logits, const torch::Tensor& targets,
                                   double smooth, int64_t background_index, double scale,
                                   double ug, double ug_min) {
  ml_params p = make_params(smooth, 1.0, scale, 1.0, background_index, ug, ug_min, 1e30, -1.0,
                            false, false, 1, 0, 0.0, -1.0, 0.0, -1.0, -1, false, true);
  return pairwise_bd_impl(logits, targets, p, true);
}

// --------------------------------------------------------------------------
// non-pairwise sigmoid CE / dice  (src/bindings.cpp:157-158,160-161)
// --------------------------------------------------------------------------
ml_dense_shape dense_shape(const torch::Tensor& logits, const torch::Tensor& targets) {
  ML_CHECK_INPUT(logits);
  ML_CHECK_INPUT(targets);
  TORCH_CHECK(logits.dim() == 5, "logits must be (L,B,C,H,W)");
  TORCH_CHECK(targets.dim() == 3, "targets must be (B,H_t,W_t)");
  TORCH_CHECK(targets.scalar_type() == torch::kLong, "targets must be int64");
  TORCH_CHECK(targets.size(0) == logits.size(1), "Batch size mismatch between logits and targets");
  TORCH_CHECK(targets.device() == logits.device(), "all tensors must be on the same device");
  ml_dense_shape s;
  s.L = logits.size(0);
  s.B = logits.size(1);
  s.C = logits.size(2);
  s.H = logits.size(3);
  s.W = logits.size(4);
  s.Ht = targets.size(1);
  s.Wt = targets.size(2);
  return s;
}

torch::Tensor dense_ws(const ml_dense_shape& s, int dt, bool dice, bool backward,
                       const torch::Tensor& like) {
  const size_t wsb = ml_dense_loss_workspace_size(&s, dt, dice, backward);
  TORCH_CHECK(wsb > 0, "unsupported shape (the target resolution must be the same integer "
                       "multiple, at most 15, of the logit resolution in both dimensions)");
  return workspace(wsb, like);
}

torch::Tensor grad_levels(const torch::Tensor& grad_out, const torch::Tensor& logits, int64_t L) {
  auto g = grad_out.to(logits.options().dtype(torch::kFloat32)).contiguous();
  TORCH_CHECK(g.numel() == L, "grad_out must have shape (L,)");
  return g;
}

torch::Tensor forward_sigmoid_ce_loss(const torch::Tensor& logits, const torch::Tensor& targets,
                                      double num_masks, double scale, double gamma, double alpha) {
  const ml_dense_shape s = dense_shape(logits, targets);
  auto loss = torch::empty({s.L}, logits.options().dtype(torch::kFloat32));
  if (s.L == 0) return loss;
  const int dt = dtype_code(logits, "logits");
  auto ws = dense_ws(s, dt, false, false, logits);
  ml_ok(ml_sigmoid_ce_forward(&s, dt, logits.data_ptr(), targets.data_ptr<int64_t>(),
                              (float)num_masks, (float)scale, (float)gamma, (float)alpha,
                              loss.data_ptr<float>(), ws.data_ptr(), ws.numel(), cur_stream()));
  return loss;
}

torch::Tensor backward_sigmoid_ce_loss(const torch::Tensor& grad_out, const torch::Tensor& logits,
                                       const torch::Tensor& targets, double num_masks,
                                       double scale, double gamma, double alpha) {
  const ml_dense_shape s = dense_shape(logits, targets);
  auto grad = torch::empty_like(logits);
  if (logits.numel() == 0) return grad;
  auto g = grad_levels(grad_out, logits, s.L);
  const int dt = dtype_code(logits, "logits");
  auto ws = dense_ws(s, dt, false, true, logits);
  ml_ok(ml_sigmoid_ce_backward(&s, dt, g.data_ptr<float>(), logits.data_ptr(),
                               targets.data_ptr<int64_t>(), (float)num_masks, (float)scale,
                               (float)gamma, (float)alpha, grad.data_ptr(), ws.data_ptr(),
                               ws.numel(), cur_stream()));
  return grad;
}

std::vector<torch::Tensor> forward_dice_loss(const torch::Tensor& logits,
                                             const torch::Tensor& targets, double smooth,
                                             double num_masks, double scale) {
  const ml_dense_shape s = dense_shape(logits, targets);
  auto f32 = logits.options().dtype(torch::kFloat32);
  auto loss = torch::empty({s.L}, f32);
  auto I = torch::empty({s.L, s.B, s.C}, f32);
  auto P = torch::empty({s.L, s.B, s.C}, f32);
  auto T = torch::empty({s.L, s.B, s.C}, f32);
  if (s.L == 0) return {loss, I, P, T};
  const int dt = dtype_code(logits, "logits");
  auto ws = dense_ws(s, dt, true, false, logits);
  ml_ok(ml_dice_loss_forward(&s, dt, logits.data_ptr(), targets.data_ptr<int64_t>(),
                             (float)smooth, (float)num_masks, (float)scale,
                             loss.data_ptr<float>(), I.data_ptr<float>(), P.data_ptr<float>(),
                             T.data_ptr<float>(), ws.data_ptr(), ws.numel(), cur_stream()));
  return {loss, I, P, T};
}

torch::Tensor backward_dice_loss(const torch::Tensor& grad_out, const torch::Tensor& logits,
                                 const torch::Tensor& targets, const torch::Tensor& I,
                                 const torch::Tensor& P, const torch::Tensor& T, double smooth,
                                 double num_masks, double scale) {
  const ml_dense_shape s = dense_shape(logits, targets);
  auto grad = torch::empty_like(logits);
  if (logits.numel() == 0) return grad;
  auto g = grad_levels(grad_out, logits, s.L);
  auto f32 = logits.options().dtype(torch::kFloat32);
  auto Ic = I.to(f32).contiguous(), Pc = P.to(f32).contiguous(), Tc = T.to(f32).contiguous();
  TORCH_CHECK(Ic.numel() == s.L * s.B * s.C && Pc.numel() == Ic.numel() && Tc.numel() == Ic.numel(),
              "I, P, T must have shape (L,B,C)");
  const int dt = dtype_code(logits, "logits");
  auto ws = dense_ws(s, dt, true, true, logits);
  ml_ok(ml_dice_loss_backward(&s, dt, g.data_ptr<float>(), logits.data_ptr(),
                              targets.data_ptr<int64_t>(), Ic.data_ptr<float>(),
                              Pc.data_ptr<float>(), Tc.data_ptr<float>(), (float)smooth,
                              (float)num_masks, (float)scale, grad.data_ptr(), ws.data_ptr(),
                              ws.numel(), cur_stream()));
  return grad;
}

// Device flag (int32, shape (1,)): 1 if any element of `x` equals `value`.
torch::Tensor any_equal(const torch::Tensor& x, int64_t value) {
  ML_CHECK_INPUT(x);
  TORCH_CHECK(x.scalar_type() == torch::kLong, "x must be int64");
  auto flag = torch::empty({1}, x.options().dtype(torch::kInt32));
  ml_ok(ml_any_equal(x.data_ptr<int64_t>(), x.numel(), value, flag.data_ptr<int32_t>(),
                     cur_stream()));
  return flag;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("pairwise_mask_loss_forward", &pairwise_mask_loss_forward,
        "Dice+Sigmoid+label pairwise cost forward (HIP, gfx950)");
  m.def("mask_matching", &mask_matching, "Mask matching: cost, assignment, loss forward (HIP)");
  m.def("mask_matching", &mask_matching_wrapper_order,
        "Mask matching, argument order used by MaskMatchingFunction (HIP)");
  m.def("mask_matching_backward", &mask_matching_backward, "Mask matching backward (HIP)");
  m.def("mask_matching_fused", &mask_matching_fused,
        "Mask matching forward that also returns the saved state for the fused backward and "
        "optionally zero-fills the gradient buffer beside the assignment (HIP)",
        py::arg("mask_logits"), py::arg("mask_targets"), py::arg("cls_logits"),
        py::arg("cls_targets"), py::arg("smooth"), py::arg("sigmoid_scale"), py::arg("dice_scale"),
        py::arg("cls_scale"), py::arg("background_index"), py::arg("uncertainty_gamma"),
        py::arg("uncertainty_gamma_min"), py::arg("inf_thresh"), py::arg("num_masks"),
        py::arg("force_unmatched_class_to_background"), py::arg("force_unmatched_masks_to_empty"),
        py::arg("topk_matches"), py::arg("strategy_id"), py::arg("mask_gamma"),
        py::arg("mask_alpha"), py::arg("cls_gamma"), py::arg("cls_alpha"),
        py::arg("void_class_index"), py::arg("use_softmax_label_loss"),
        py::arg("normalize_uncertainty"), py::arg("grad_prefill") = py::none(),
        py::arg("check_void") = false);
  m.def("mask_matching_autograd", &mask_matching_autograd,
        "MaskMatchingFunction's forward as a C++ autograd node: pred_to_gt, pred_round and the "
        "three layer means, differentiable in the mask and class logits (HIP)",
        py::arg("mask_logits"), py::arg("mask_targets"), py::arg("cls_logits"),
        py::arg("cls_targets"), py::arg("smooth"), py::arg("sigmoid_scale"), py::arg("dice_scale"),
        py::arg("cls_scale"), py::arg("background_index"), py::arg("uncertainty_gamma"),
        py::arg("uncertainty_gamma_min"), py::arg("inf_thresh"), py::arg("num_masks"),
        py::arg("force_unmatched_class_to_background"), py::arg("force_unmatched_masks_to_empty"),
        py::arg("topk_matches"), py::arg("strategy_id"), py::arg("mask_gamma"),
        py::arg("mask_alpha"), py::arg("cls_gamma"), py::arg("cls_alpha"),
        py::arg("void_class_index"), py::arg("use_softmax_label_loss"),
        py::arg("normalize_uncertainty"), py::arg("check_void") = false);
  m.def("mask_matching_backward_fused", &mask_matching_backward_fused,
        "Mask matching backward using the forward's saved state (HIP)", py::arg("g_mask"),
        py::arg("g_dice"), py::arg("g_cls"), py::arg("mask_logits"), py::arg("mask_targets"),
        py::arg("cls_logits"), py::arg("cls_targets"), py::arg("pred_to_gt"), py::arg("smooth"),
        py::arg("sigmoid_scale"), py::arg("dice_scale"), py::arg("cls_scale"),
        py::arg("background_index"), py::arg("uncertainty_gamma"),
        py::arg("uncertainty_gamma_min"), py::arg("num_masks"),
        py::arg("force_unmatched_class_to_background"), py::arg("force_unmatched_masks_to_empty"),
        py::arg("mask_gamma"), py::arg("mask_alpha"), py::arg("cls_gamma"), py::arg("cls_alpha"),
        py::arg("void_class_index"), py::arg("use_softmax_label_loss"),
        py::arg("normalize_uncertainty"), py::arg("saved"), py::arg("grad_prefill") = py::none());
  m.def("forward_pw_sigmoid_label_loss", &forward_pw_sigmoid_label_loss,
        "Pairwise sigmoid label cost forward (HIP)");
  m.def("forward_pw_softmax_label_loss", &forward_pw_softmax_label_loss,
        "Pairwise softmax label cost forward (HIP)");
  m.def("forward_sigmoid_ce_loss", &forward_sigmoid_ce_loss, "Sigmoid cross entropy forward (HIP)");
  m.def("backward_sigmoid_ce_loss", &backward_sigmoid_ce_loss,
        "Sigmoid cross entropy backward (HIP)");
  m.def("forward_pw_sigmoid_ce_loss", &forward_pw_sigmoid_ce_loss,
        "Pairwise sigmoid cross entropy forward (HIP)");
  m.def("forward_dice_loss", &forward_dice_loss, "Dice loss forward (HIP)");
  m.def("backward_dice_loss", &backward_dice_loss, "Dice loss backward (HIP)");
  m.def("forward_pw_dice_loss", &forward_pw_dice_loss, "Pairwise dice loss forward (HIP)");
  m.def("point_sample", &point_sample, "Bilinear point sampling, grid_sample semantics (HIP)");
  m.def("point_sample_backward", &point_sample_backward,
        "Gradient of point_sample with respect to its input (HIP)");
  m.def("point_sample_masks", &point_sample_masks,
        "Bilinear point sampling of (L,B,Q,H,W) logits at (B,P,2) points (HIP)");
  m.def("point_labels", &point_labels, "Labels under (B,P,2) points, floor mapping (HIP)");
  m.def("forward_pw_sigmoid_ce_loss_sampling", &forward_pw_sigmoid_ce_loss_sampling,
        "Pairwise sigmoid CE over sampled points (HIP)");
  m.def("forward_pw_dice_loss_sampling", &forward_pw_dice_loss_sampling,
        "Pairwise dice loss over sampled points (HIP)");
  m.def("any_equal", &any_equal, "Device flag: any element equal to value (HIP)");
  m.attr("__backend__") = "hip-gfx950";
}
