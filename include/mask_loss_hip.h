/*
 * mask_loss_hip.h -- C ABI of the MI355X (gfx950) mask-cost / assignment /
 * matched-loss library (libmask_loss_hip.so).
 *
 * Plain pointers, sizes and a hipStream_t; no framework types.  Every entry
 * point enqueues work on `stream` and returns without synchronising (except
 * ml_mask_matching_forward_polled, which waits for its forward's second
 * kernel before it queues the rest).  All
 * device pointers must be device-accessible, contiguous, row-major.
 * Return value: ML_OK (0) or an ML_E* code; ml_last_error() returns the
 * message of the last failure on the calling thread.
 *
 * Scratch memory is never allocated inside: callers query the size with the
 * matching *_workspace_size() function and pass a device buffer of at least
 * that many bytes (256-byte aligned).
 *
 * Reference interface replaced by each entry point (AndyBarcia/mask_loss):
 *   ml_pairwise_mask_loss_forward   src/cuda/pw_mask.cu:314-501
 *                                   (bound at src/bindings.cpp:164)
 *   ml_mask_matching_forward        src/cpu/matching.cpp:592-752
 *                                   (bound at src/bindings.cpp:165)
 *   ml_mask_matching_backward       src/cuda/mask_matching_backward.cu:378-621
 *                                   (bound at src/bindings.cpp:166)
 *   ml_pairwise_label_loss_forward  src/cuda/pw_sigmoid_label_loss.cu:108-187 and
 *                                   src/cuda/pw_softmax_label_loss.cu:105-173
 *                                   (bound at src/bindings.cpp:167-168)
 *   ml_pairwise_sigmoid_dice_forward src/cuda/pw_sigmoid_ce.cu:199-316 and
 *                                   src/cuda/pw_dice_loss.cu:111-221
 *                                   (bound at src/bindings.cpp:159,162)
 *   ml_sigmoid_ce_forward/backward  src/cuda/sigmoid_ce.cu:207-332
 *                                   (bound at src/bindings.cpp:157-158)
 *   ml_dice_loss_forward/backward   src/cuda/dice_loss.cu:159-289
 *                                   (bound at src/bindings.cpp:160-161)
 *   ml_point_sample(_backward)      functions/utils.py:12-20 (point_sample, through
 *                                   F.grid_sample and its input gradient)
 *   ml_point_labels                 functions/sigmoid/pw_sigmoid_ce.py:497-502
 *   ml_pairwise_sigmoid_dice_points_forward
 *                                   functions/sigmoid/pw_sigmoid_ce.py:407-550 and
 *                                   functions/dice/pw_dice_loss.py:174-268
 *                                   (the *_sampling_py costs, for given points)
 */
#ifndef MASK_LOSS_HIP_H
#define MASK_LOSS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* ml_stream_t; /* == hipStream_t */
typedef struct ihipEvent_t* ml_event_t;   /* == hipEvent_t */

enum {
  ML_OK = 0,
  ML_EINVAL = 1,     /* invalid argument (shape, range, flag combination) */
  ML_EWORKSPACE = 2, /* workspace too small */
  ML_ELAUNCH = 3,    /* HIP launch / runtime error */
  ML_EUNSUPPORTED = 4
};

enum { ML_F32 = 0, ML_BF16 = 1, ML_F16 = 2 };

/* Strategy ids, reference src/cpu/matching.cpp:60-65. */
enum { ML_GLOBAL = 0, ML_ROUND = 1, ML_GREEDY = 2, ML_PSEUDO_GREEDY = 3 };

/* Shapes of one call.  mask logits (L,B,Q,H,W); targets (B,Ht,Wt) int64 label
 * map; cls logits (L,B,Q,C); cls targets (B,GT_total) int64 (-1 padding). */
typedef struct ml_shape {
  int64_t L, B, Q, H, W, Ht, Wt, C, GT_total;
} ml_shape;

/* Loss / matching options; field meaning follows the positional arguments of
 * mask_matching (src/bindings.cpp:84-111, src/cpu/matching.cpp:592-617). */
typedef struct ml_params {
  float smooth, sigmoid_scale, dice_scale, cls_scale;
  int64_t background_index;
  float uncertainty_gamma, uncertainty_gamma_min;
  double inf_thresh, num_masks;
  int32_t force_unmatched_class_to_background;
  int32_t force_unmatched_masks_to_empty;
  int64_t topk_matches, strategy_id;
  float mask_gamma, mask_alpha, cls_gamma, cls_alpha;
  int64_t void_class_index;
  int32_t use_softmax_label_loss;
  int32_t normalize_uncertainty;
} ml_params;

/* State the fused forward leaves for the backward ("saved": ml_saved_bytes()
 * bytes, 256-byte aligned, written by ml_mask_matching_forward, read by
 * ml_mask_matching_backward).  Its head is float: per-query statistics
 * stats[(l*B+b)*Q+q][ML_STAT_*], then the per-layer block layer[l][ML_LAYER_*];
 * after them (internal layout) the list of matched query rows and, when the
 * targets are at the logit resolution, the compact label map, so the backward
 * neither recomputes statistics nor re-reads the int64 label map. */
enum {
  ML_STAT_S = 0,    /* uncertainty normaliser after normalise/clamp */
  ML_STAT_P = 1,    /* sum_j N2 w p */
  ML_STAT_I = 2,    /* sum_j w p n  for the matched GT (0 if unmatched) */
  ML_STAT_T = 3,    /* sum_j w n    for the matched GT (0 if unmatched) */
  ML_STATS = 4
};
enum { ML_LAYER_INV_MASK_DEN = 0, ML_LAYER_INV_CLS_DEN = 1, ML_LAYERS = 2 };
size_t ml_saved_bytes(const ml_shape* s, const ml_params* p, int mask_dtype);

const char* ml_last_error(void);
int ml_version(void);

/* ---- pairwise mask + label cost (3, L, B, Q, GT_out) float ---------------- */
size_t ml_pairwise_mask_loss_workspace_size(const ml_shape* s, const ml_params* p,
                                            int mask_dtype);
int ml_pairwise_mask_loss_forward(const ml_shape* s, const ml_params* p,
                                  int mask_dtype, const void* mask_logits,
                                  const int64_t* mask_targets, int cls_dtype,
                                  const void* cls_logits, const int64_t* cls_targets,
                                  float* separate_costs, void* workspace,
                                  size_t workspace_bytes, ml_stream_t stream);

/* ---- full matching forward: costs -> assignment -> per-layer means -------- */
size_t ml_mask_matching_workspace_size(const ml_shape* s, const ml_params* p,
                                       int mask_dtype);
/* pred_to_gt / pred_round: (L,B,Q) int64; layer_means: (3,L) float
 * [mask, dice, cls]; separate_costs: (3,L,B,Q,GT_out) float or NULL;
 * saved: ml_saved_bytes() bytes for the backward, or NULL.
 * grad_mask_prefill: NULL, or the (L,B,Q,H,W) mask_dtype buffer (16-byte
 * aligned) that will receive the mask-logit gradient.  The forward then
 * zero-fills it with extra workgroups of the assignment launch (the
 * assignment occupies one CU per image and leaves HBM idle), and the backward
 * called with grad_prefilled = 1 writes only the matched rows.  Not allowed
 * with force_unmatched_masks_to_empty (every row has a gradient then).
 * void_found: NULL, or an int32 the device can write (device memory, or
 * pinned host memory mapped for the device): it receives 1 if any of the
 * B*GT_total entries of cls_targets equals params.void_class_index (a valid
 * class index), else 0 -- the reference's check of
 * functions/mask/matching.py:184-185, done by the forward's first kernels
 * with a system-scope store, so a host can poll a coherent pinned word
 * (preset to another value) without waiting for the whole forward.
 * void_ready: NULL, or a hipEvent_t recorded on `stream` as soon as
 * void_found is written (before the cost contraction); recording it costs
 * the next kernel a system-scope release, so polling is the faster wait. */
int ml_mask_matching_forward(const ml_shape* s, const ml_params* p, int mask_dtype,
                             const void* mask_logits, const int64_t* mask_targets,
                             int cls_dtype, const void* cls_logits,
                             const int64_t* cls_targets, int64_t* pred_to_gt,
                             int64_t* pred_round, float* layer_means,
                             float* separate_costs, void* saved, void* grad_mask_prefill,
                             int32_t* void_found, ml_event_t void_ready,
                             void* workspace, size_t workspace_bytes, ml_stream_t stream);

/* ---- matching forward that skips empty column classes --------------------------
 * No counterpart in the reference: for a host thread that can wait while its
 * kernels run (the library's own PyTorch binding uses it).  The forward of
 * ml_mask_matching_forward, same arguments and results, plus the device and
 * host addresses of three int32 words of pinned, coherent host memory mapped
 * for the device.  The cost contraction runs one launch per column-tile class
 * (images with up to 31, 111 and 255 non-empty GTs), and which classes have
 * images is known on the device only, so ml_mask_matching_forward launches
 * every class that the shape allows; an empty launch still costs the GPU a
 * few microseconds.  Here the forward's column pass stores each class's task
 * count into the words (system-scope stores); the call queues one class
 * unconditionally (the narrowest when the shape allows two classes, the
 * widest when it allows three), waits for the counts (polling; after 2 s it
 * synchronizes the stream) while that class runs, queues only the other
 * classes that have tasks, then the rest of the forward, and returns while
 * that runs.  When the widest class and another class both have images, the
 * widest class's assignment runs on a second stream of the library's own
 * (default priority, forked from and joined back into `stream` by events),
 * beside the other classes' contraction; work queued on `stream` after the
 * call follows it.  Not for graph capture (the wait
 * needs the kernels to run), and one call at a time per set of words.
 * ML_EINVAL if either address is null. */
int ml_mask_matching_forward_polled(const ml_shape* s, const ml_params* p, int mask_dtype,
                                    const void* mask_logits, const int64_t* mask_targets,
                                    int cls_dtype, const void* cls_logits,
                                    const int64_t* cls_targets, int64_t* pred_to_gt,
                                    int64_t* pred_round, float* layer_means, float* separate_costs,
                                    void* saved, void* grad_mask_prefill, int32_t* void_found,
                                    ml_event_t void_ready, void* workspace, size_t workspace_bytes,
                                    ml_stream_t stream, int32_t* class_counts_dev,
                                    volatile int32_t* class_counts_host);

/* ---- matching forward without allocation -------------------------------------
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  ml_mask_matching_forward with the same arguments and
 * results, minus workspace / workspace_bytes: its scratch is a static device
 * array of ML_NOALLOC_SCRATCH_BYTES (128 MiB) on each device it runs on, held
 * until the process ends; the call itself allocates and frees nothing.
 * Shapes that need more scratch than that fail with ML_EUNSUPPORTED (the
 * headline shape, B=16, Q=200, 256x256, up to 100 GT columns, fits).  Calls
 * that overlap on one device share the array and race: serialise them (one
 * stream, or wait between calls).  The array's contents need no clearing
 * between calls. */
#define ML_NOALLOC_SCRATCH_BYTES ((size_t)128 << 20)
int ml_mask_matching_forward_noalloc(const ml_shape* s, const ml_params* p, int mask_dtype,
                                     const void* mask_logits, const int64_t* mask_targets,
                                     int cls_dtype, const void* cls_logits,
                                     const int64_t* cls_targets, int64_t* pred_to_gt,
                                     int64_t* pred_round, float* layer_means,
                                     float* separate_costs, void* saved, void* grad_mask_prefill,
                                     int32_t* void_found, ml_event_t void_ready,
                                     ml_stream_t stream);
/* Scratch bytes ml_mask_matching_forward_noalloc needs for this shape on the
 * current device (its cost plan is sized for the device's resident waves),
 * to compare with ML_NOALLOC_SCRATCH_BYTES before a call; 0 on an invalid
 * or unsupported shape (ml_last_error() says why).  No counterpart in the
 * reference; allocates nothing and launches nothing. */
size_t ml_mask_matching_forward_noalloc_bytes(const ml_shape* s, const ml_params* p, int mask_dtype);

/* ---- matching backward ------------------------------------------------------
 * grad_{mask,dice,cls}: (L,) float upstream gradients of the layer means.
 * grad_mask_logits: (L,B,Q,H,W) in mask_dtype; grad_cls_logits: (L,B,Q,C) in
 * cls_dtype.  saved == NULL recomputes the per-query statistics from the
 * logits (the reference's two-pass backward); otherwise the state saved by
 * ml_mask_matching_forward is used and each matched logit is read once.
 * grad_prefilled = 1 (requires `saved`): grad_mask_logits is the buffer the
 * forward zero-filled, and only matched rows are written. */
size_t ml_mask_matching_backward_workspace_size(const ml_shape* s, const ml_params* p,
                                                int mask_dtype);
int ml_mask_matching_backward(const ml_shape* s, const ml_params* p,
                              const float* grad_mask, const float* grad_dice,
                              const float* grad_cls, int mask_dtype,
                              const void* mask_logits, const int64_t* mask_targets,
                              int cls_dtype, const void* cls_logits,
                              const int64_t* cls_targets, const int64_t* pred_to_gt,
                              const void* saved, int grad_prefilled, void* grad_mask_logits,
                              void* grad_cls_logits, void* workspace,
                              size_t workspace_bytes, ml_stream_t stream);

/* ---- pairwise label cost (L,B,Q,GT_out) float; use_softmax selects the
 * softmax-CE form, otherwise sigmoid-BCE with (gamma, alpha). -------------- */
int ml_pairwise_label_loss_forward(int64_t L, int64_t B, int64_t Q, int64_t C,
                                   int64_t GT_total, int cls_dtype,
                                   const void* cls_logits, const int64_t* cls_targets,
                                   int64_t background_index, float scale, float gamma,
                                   float alpha, int use_softmax, float* out,
                                   ml_stream_t stream);

/* ---- standalone pairwise sigmoid-BCE and dice costs (L,B,C,GT_out) float ----
 * logits (L,B,C,H,W) as mask logits with s->Q = C channels; s->GT_total = the
 * number of label slots (the reference takes targets.max()+1,
 * src/cuda/pw_sigmoid_ce.cu:222-224, src/cuda/pw_dice_loss.cu:132-134);
 * s->C and the class fields of `p` are unused.  bce_out / dice_out may each
 * be NULL.  Fields used: background_index, sigmoid_scale (BCE scale),
 * dice_scale (dice scale), smooth, mask_gamma / mask_alpha (BCE focal),
 * uncertainty_gamma(_min), normalize_uncertainty (BCE).  Workspace: the
 * size ml_pairwise_mask_loss_workspace_size() returns for the same shape.
 * Replaces src/cuda/pw_sigmoid_ce.cu:199-316 (bound at src/bindings.cpp:159)
 * and src/cuda/pw_dice_loss.cu:111-221 (bound at src/bindings.cpp:162). */
int ml_pairwise_sigmoid_dice_forward(const ml_shape* s, const ml_params* p, int dtype,
                                     const void* logits, const int64_t* targets,
                                     float* bce_out, float* dice_out, void* workspace,
                                     size_t workspace_bytes, ml_stream_t stream);

/* ---- point-sampling front end (Mask2Former-style matching on sampled points)
 * ml_point_sample: out[n][c][p] = bilinear sample of input plane (n, c) at
 *   coords[n % coords_batch][p] = (x, y) in [0, 1], i.e. grid_sample(input,
 *   2 * coords - 1, mode bilinear, zero padding, align_corners); input
 *   (N,C,H,W) and out (N,C,P) in `dtype`, coords float (coords_batch,P,2).
 *   Replaces point_sample, functions/utils.py:12-20 (F.grid_sample), as
 *   called at functions/sigmoid/pw_sigmoid_ce.py:489-495 and
 *   functions/dice/pw_dice_loss.py:235-239 (coords shared by every (L, C)
 *   map of an image: N = L*B, C = queries, coords_batch = B).
 * ml_point_labels: labels[b][p] = targets[b][iy][ix] with
 *   ix = clamp(long(x * (Wt-1)), 0, Wt-1) in float32 (NaN -> 0), likewise iy;
 *   targets (B,Ht,Wt) int64, labels (B,P) int64.  Replaces the nearest-label
 *   lookup of functions/sigmoid/pw_sigmoid_ce.py:497-502 and
 *   functions/dice/pw_dice_loss.py:242-245.
 * ml_pairwise_sigmoid_dice_points_forward: the pairwise sigmoid-BCE / dice
 *   costs of ml_pairwise_sigmoid_dice_forward over P sampled points:
 *   point_logits (L,B,C,1,P) in `dtype` (ml_point_sample's output), with
 *   s->H = s->Ht = 1, s->W = s->Wt = P, s->Q = C, s->GT_total = the label
 *   slots (the reference: max of the full map + 1); the labels under
 *   `coords` (B,P,2) in the full map targets (B,Hs,Ws) are the binary
 *   targets, and a GT is present (finite costs) iff it has a pixel anywhere in
 *   the full map.  With uncertainty_gamma = 0 and normalize_uncertainty = 0
 *   this is the reference's pairwise_sigmoid_cross_entropy_loss_sampling_py
 *   (functions/sigmoid/pw_sigmoid_ce.py:407-550) and
 *   pairwise_dice_loss_sampling_py (functions/dice/pw_dice_loss.py:174-268)
 *   for given points.  Workspace from ml_pairwise_points_workspace_size. */
int ml_point_sample(int dtype, const void* input, const float* coords, int64_t N, int64_t C,
                    int64_t H, int64_t W, int64_t P, int64_t coords_batch, int align_corners,
                    void* out, ml_stream_t stream);
/* ml_point_sample_backward: grad_input (N,C,H,W) = the gradient of
 *   ml_point_sample with respect to its input, for grad_out (N,C,P), both in
 *   `dtype`: each sample's gradient added to its four corner cells with its
 *   bilinear weights (grid_sample's input gradient, functions/utils.py:17).
 *   A cell's contributions are summed in float32 in an order that can change
 *   between runs, as with the reference's CUDA grid_sample backward (float
 *   atomics).  Every cell of grad_input is written.  Workspace:
 *   ml_point_sample_backward_workspace_size bytes for the same shape,
 *   P and coords_batch (0 for some shapes). */
size_t ml_point_sample_backward_workspace_size(int dtype, int64_t N, int64_t C, int64_t H,
                                               int64_t W, int64_t P, int64_t coords_batch);
int ml_point_sample_backward(int dtype, const void* grad_out, const float* coords, int64_t N,
                             int64_t C, int64_t H, int64_t W, int64_t P, int64_t coords_batch,
                             int align_corners, void* grad_input, float* workspace,
                             size_t workspace_bytes, ml_stream_t stream);
int ml_point_labels(const int64_t* targets, const float* coords, int64_t B, int64_t Ht,
                    int64_t Wt, int64_t P, int64_t* labels, ml_stream_t stream);
size_t ml_pairwise_points_workspace_size(const ml_shape* s, const ml_params* p, int dtype,
                                         int64_t Hs, int64_t Ws);
int ml_pairwise_sigmoid_dice_points_forward(const ml_shape* s, const ml_params* p, int dtype,
                                            const void* point_logits, const int64_t* targets,
                                            int64_t Hs, int64_t Ws, const float* coords,
                                            float* bce_out, float* dice_out, void* workspace,
                                            size_t workspace_bytes, ml_stream_t stream);

/* ---- non-pairwise sigmoid-CE and dice losses over dense class logits --------
 * logits (L,B,C,H,W) in `dtype`, targets (B,Ht,Wt) int64 class labels
 * (labels outside [0,C) count for no class).  Workspace from
 * ml_dense_loss_workspace_size(s, dtype, dice, backward).
 *   ml_sigmoid_ce_forward   src/cuda/sigmoid_ce.cu:207-268  (src/bindings.cpp:157)
 *   ml_sigmoid_ce_backward  src/cuda/sigmoid_ce.cu:270-332  (src/bindings.cpp:158)
 *   ml_dice_loss_forward    src/cuda/dice_loss.cu:159-222   (src/bindings.cpp:160)
 *   ml_dice_loss_backward   src/cuda/dice_loss.cu:224-289   (src/bindings.cpp:161)
 * loss: (L,) float; I, P, T: (L,B,C) float; grad_out: (L,) float; grad: (L,B,C,H,W)
 * in `dtype`.  Sums are float64 and reduced in a fixed order. */
typedef struct ml_dense_shape {
  int64_t L, B, C, H, W, Ht, Wt;
} ml_dense_shape;
size_t ml_dense_loss_workspace_size(const ml_dense_shape* s, int dtype, int dice, int backward);
int ml_sigmoid_ce_forward(const ml_dense_shape* s, int dtype, const void* logits,
                          const int64_t* targets, float num_masks, float scale, float gamma,
                          float alpha, float* loss, void* workspace, size_t workspace_bytes,
                          ml_stream_t stream);
int ml_sigmoid_ce_backward(const ml_dense_shape* s, int dtype, const float* grad_out,
                           const void* logits, const int64_t* targets, float num_masks,
                           float scale, float gamma, float alpha, void* grad, void* workspace,
                           size_t workspace_bytes, ml_stream_t stream);
int ml_dice_loss_forward(const ml_dense_shape* s, int dtype, const void* logits,
                         const int64_t* targets, float smooth, float num_masks, float scale,
                         float* loss, float* I, float* P, float* T, void* workspace,
                         size_t workspace_bytes, ml_stream_t stream);
int ml_dice_loss_backward(const ml_dense_shape* s, int dtype, const float* grad_out,
                          const void* logits, const int64_t* targets, const float* I,
                          const float* P, const float* T, float smooth, float num_masks,
                          float scale, void* grad, void* workspace, size_t workspace_bytes,
                          ml_stream_t stream);

/* ---- input validation helper ------------------------------------------------
 * flag[0] = 1 if any of x[0..n) equals `value`, else 0 (one small kernel, no
 * synchronisation).  Replaces the device-wide comparison + reduction behind
 * the reference's void-class check (functions/mask/matching.py:184-185), so
 * the caller can read the flag asynchronously. */
int ml_any_equal(const int64_t* x, int64_t n, int64_t value, int32_t* flag, ml_stream_t stream);

/* ---- instrumentation (no counterpart in the reference) ---------------------
 * When enabled, every kernel launch of this library is bracketed by HIP events
 * recorded on its own stream.  ml_profile_read() waits for those events and
 * returns, for kernel family `name` ("prep", "pair_cost", "assign", "layer",
 * "bwd_mask", "bwd_cls", "label_cost", "prefill"), the number of launches and their
 * summed duration in milliseconds since the last reset. */
int ml_profile_enable(int enable);
int ml_profile_read(const char* name, int64_t* launches, double* total_ms);
int ml_profile_reset(void);

/* Measurement aid (no counterpart in the reference): a read-only HBM stream
 * over `bytes` bytes at `p` (16-byte aligned, bytes a multiple of 16) by
 * `grid` workgroups of 256 threads, each reading one contiguous chunk with
 * 16-byte loads (eight in flight per thread) and writing one word to
 * out[blockIdx] -- the practical read ceiling that the cost contraction,
 * which streams every logit once, is measured against. */
int ml_profile_stream_read(const void* p, size_t bytes, uint32_t* out, int grid,
                           ml_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MASK_LOSS_HIP_H */
