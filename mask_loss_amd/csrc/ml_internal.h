// Host-side launch plumbing shared by the kernels' translation units:
// workspace layout, kernel argument blocks, launcher declarations.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <mutex>
#include <string>

#include "ml_common.h"

namespace ml {

// bf16 per-cell terms from LDS tables (1, default) or from the formulas (0, tests).
extern int g_use_lut;

// Set the thread-local error message returned by ml_last_error().
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

constexpr int kStep = 32;        // cells per MFMA K-step (16x16x32)
// Presence bits per image: make_dims admits at most 255 GT columns, so the
// forward's GT labels are < 256.
constexpr int kPresWords = 8;
constexpr int kPresLabels = 32 * kPresWords;
// Workgroups of 256 threads that zero-fill the gradient buffer beside the
// assignment (measured on MI355X: 64 still write at the full rate while
// leaving the other CUs to the latency-bound assignment).
constexpr int kFillBlocks = 64;
// Slices of that fill given instead to the preparation's column pass and to
// the finalize launch, as extra workgroups beside their own work: both are
// short, latency-bound launches that leave HBM nearly idle, so these bytes
// come off the assignment launch, where the fill outlasts a short assignment.
// (The column pass takes none when the shape allows three column-tile
// classes: the split forward's critical path waits for that pass.)
constexpr int64_t kPrepFillBytes = (int64_t)56 << 20;
constexpr int64_t kFinFillBytes = (int64_t)16 << 20;

// Column-tile classes of the cost contraction: an image with G non-empty GT
// columns (+ the ones column) is handled by the kernel instance whose tile
// count NT is the smallest of {2, 7, 16} that holds G + 1 columns.  Which
// classes have images is known on the device only, and every class launch
// costs its dispatch latency even when empty, so the classes are few.
constexpr int kClasses = 3;
__host__ __device__ inline int class_nt(int ci) { return ci == 0 ? 2 : ci == 1 ? 7 : 16; }
// Waves per cost workgroup (all share one LDS table): 16 for the narrowest
// class on the table path (one workgroup per CU, at most 128 registers per
// lane), 4 for the widest class (its accumulators need more than 256
// registers per lane), 8 otherwise.
__host__ __device__ constexpr int cost_waves(int nt, bool tab) {
  return nt == 2 && tab ? 16 : nt >= 16 ? 4 : 8;
}
__host__ __device__ inline int class_of(int ncols_plus_one) {
  const int need = (ncols_plus_one + 15) >> 4;
  return need <= 2 ? 0 : need <= 7 ? 1 : 2;
}
// Whether an image with G non-empty columns belongs to a launch restricted to
// the image subset (phase_class, phase_in) (see AssignArgs).
__host__ __device__ inline bool in_phase(int phase_class, int phase_in, int G) {
  return phase_class < 0 || ((class_of(G + 1) == phase_class) == (phase_in != 0));
}
// Upper bound of resident cost waves the workspace is sized for (256 CUs x 16).
constexpr int64_t kCostSlots = 4096;
// CUs the narrower classes' cost launches leave free, with three classes, for
// the widest class's assignment (at most one per image, at most 1/8 of them)
constexpr int kSideCUs = 16;

// Host-side plan of the cost launches.  Each class launch has `slots[c]`
// waves (what the GPU holds resident at that kernel's occupancy, at most
// kCostSlots); on the device the schedule picks the class's K-split KS_c =
// clamp(slots / n_c, 1, ks_max) for its n_c (image, row-tile) tasks, and wave
// w of the class takes task w / KS_c, split w % KS_c (grid-stride beyond).
// Classes 1 and 2 may instead split each task R_c times finer and add R_c
// consecutive splits in the workgroup (see the cost kernel), so that KS_c
// partials per task remain.  Work item w of class c (task i, partial k:
// w = k * n_c + i) owns partial tile float_base[c] + w * tile(c) and global
// slot slot_base[c] + w (unweighted row sums).
struct CostPlan {
  int nclass;                    // classes with class_nt(c) <= padded NT
  int slots[kClasses];
  int64_t slot_base[kClasses];
  int64_t float_base[kClasses];
  int64_t ks_max;
  int64_t ntasks;                // L * B * rtiles
  int64_t float_total;           // partials size (floats)
  int64_t slot_total;            // work-item slots of all classes (row-sum records)
  int64_t rtiles;                // row tiles per image
  // Class 0 runs as row-tile pairs: a wave takes row tiles 2k and 2k + 1 of
  // one image (32 query rows, 32x32x16 products), its work item is pair k of
  // the class's images at one K-split, and its partial tile holds both row
  // tiles ([3][2 rows][nslot]).  No row-sum records on this path.
  int pair0;
  // Planes per partial tile of each class: 3 (bce numerator, I, T) or 4 for
  // classes 1 and 2 on label maps without the bf16 table (per-slot sums of
  // A_neg, A_pos, A_p, A_w over the cells whose label is that slot's column;
  // slot G holds the cells of no column).  Finalize rebuilds the bce
  // numerator of slot g as the sum of the other slots' A_neg sums plus g's
  // A_pos sum, and P, S as the sums over all slots.
  int planes[kClasses];
};
// Device schedule (ints in the workspace): n[kClasses], ks[kClasses] (the
// K-split partials of each task that reach the partial sums), red[kClasses]
// (waves per partial: each partial is the sum of red consecutive K-splits,
// added in the workgroup; 1 for class 0), list[kClasses][ntasks] (task ids per
// class, ascending), idx[ntasks] (position of each task in its class list).
constexpr int kSchedRed = 2 * kClasses;
constexpr int kSchedList = 3 * kClasses;
__host__ __device__ inline int64_t sched_ints(int64_t ntasks) { return kSchedList + (kClasses + 1) * ntasks; }

// Work item w of column-tile class c (n_c tasks, KS_c splits) is task
// i = w % n_c at K-split ks = w / n_c: consecutive waves take consecutive row
// tiles at the same K offset, so the rows a workgroup streams are adjacent.
// Item w owns partial tile float_base[c] + w * tile and row-sum slot
// slot_base[c] + w.
//
// Where the K-split partial sums of query row (lb, q) live: split 0's value
// of plane 0 at column slot 0, the stride between splits and between planes,
// the split count, and the row-sum slot of split 0 and the stride between
// splits' slots.
struct RowPartials {
  const float* p0;
  int64_t ks_stride, plane, slot0, slot_stride;
  int KS;
};
// The same from values already loaded: the row's column class ci, the task's
// index i within that class's list of n tasks, the class's split count KS
// and the row's index qin within its row tile.
__device__ inline RowPartials row_partials_at(const float* partials, const CostPlan& plan, int ci,
                                              int64_t i, int KS, int64_t n, int qin, int64_t rows) {
  const int64_t nslot_c = 16 * class_nt(ci);
  const int64_t tile = plan.planes[ci] * rows * nslot_c;
  RowPartials r;
  r.KS = KS;
  if (ci == 0 && plan.pair0) {
    // task i = row tile rt of the class's j-th image; pair j * prt + rt / 2
    // of the np pairs, row tile rt & 1 within it
    const int64_t prt = (plan.rtiles + 1) >> 1;
    const int64_t j = i / plan.rtiles, rt = i - j * plan.rtiles;
    const int64_t p = j * prt + (rt >> 1), np = (n / plan.rtiles) * prt;
    r.ks_stride = np * 2 * tile;
    r.plane = 2 * rows * nslot_c;
    r.p0 = partials + plan.float_base[0] + p * 2 * tile + ((rt & 1) * rows + qin) * nslot_c;
    r.slot0 = plan.slot_base[0] + p;
    r.slot_stride = np;
    return r;
  }
  r.ks_stride = n * tile;
  r.plane = rows * nslot_c;
  r.p0 = partials + plan.float_base[ci] + i * tile + qin * nslot_c;
  r.slot0 = plan.slot_base[ci] + i;
  r.slot_stride = n;
  return r;
}

// Derived sizes of one call.
struct Dims {
  int64_t L, B, Q, H, W, Ht, Wt, C, GT_total;
  int64_t LB, HW, s, N2;
  int64_t GT_out, bg;        // compacted column count, normalised background slot
  int64_t HWp;               // HW padded to a multiple of kStep
  int NT;                    // 16-wide column tiles (valid GT columns + ones column)
  int RT;                    // 16-row tiles per wave
  int rows;                  // rows per cost workgroup (16 * RT)
  int64_t rtiles;            // row tiles per image
  int64_t ks_max;            // most K-splits per task (>= 8 K-steps per wave)
  int nslot;                 // 16 * NT
  bool counts_mode;          // s > 1: per-cell count operands
  int cw;                    // bytes per count: 1 (u8, s <= 15) or 2 (u16, s >= 16)
  bool pair_ok;              // bf16 label maps whose rows suit the row-tile pair kernel
};

bool make_dims(const ml_shape* s, int64_t background_index, int dtype, Dims& d, std::string& err);
int cost_rt_for(int dtype, int NT);

// Byte offsets inside the forward's saved state (see ml_saved_bytes): the
// float head (per-query stats, then the per-layer block), the matched-row list
// (int32 count, then (l*B+b)*Q+q of every matched row, ascending), and for
// s == 1 the compact label map lab16 [B][HWp].
struct SavedLayout {
  size_t stats, layer, list, lab16, total;
};
inline SavedLayout saved_layout(const Dims& d) {
  SavedLayout S;
  S.stats = 0;
  S.layer = (size_t)d.LB * d.Q * ML_STATS * 4;
  S.list = align256(S.layer + (size_t)d.L * ML_LAYERS * 4);
  S.lab16 = align256(S.list + (size_t)(1 + d.LB * d.Q) * 4);
  S.total = align256(S.lab16 + (d.counts_mode ? 0 : (size_t)d.B * d.HWp * 2));
  return S;
}

// Byte offsets inside the caller's workspace.
struct Layout {
  size_t lab16, counts, pbits, ncols, colmap, slot_of_col, sched, partials, rowsum,
      sep, tot, tot64, rowIT, rowstat, img, mrows, layer, done, total;
};
// Workspace layout for the cost plan `pl` (its float_total / slot_total size
// the partial-sum regions).
Layout make_layout(const Dims& d, bool force_masks, const CostPlan& pl);
Layout make_layout(const Dims& d, bool force_masks);  // with bound_cost_plan(d)
// Plan slots / offsets of the cost launches (queries kernel occupancy on the
// current device; the workspace bound uses kCostSlots only).
CostPlan make_cost_plan(const Dims& d, int dtype, bool tab);
CostPlan bound_cost_plan(const Dims& d);
// Region offsets re-packed for the plan's own slot counts (class c holds
// max(slots[c], ntasks) work items): the smallest layout that gives the same
// K-splits, and so the same results, as the bound layout.
void pack_cost_plan(CostPlan& p, const Dims& d);
// pack_cost_plan, with fewer slots for the classes with the largest partial
// regions until the layout fits `budget` bytes (or no class can shrink)
void fit_cost_plan(CostPlan& p, const Dims& d, bool force_masks, size_t budget);

// ---- kernel argument blocks ------------------------------------------------
// Part of the gradient's zero fill done by `blocks` extra workgroups of a
// launch: 16-byte words [0, n16) from p.
struct FillSlice {
  u32x4_t* p = nullptr;
  int64_t n16 = 0;
  int blocks = 0;
};

struct PrepArgs {
  const int64_t* targets;
  uint16_t* lab16;
  uint8_t* counts;       // s > 1: [B][GT_total][HWp] counts of cw bytes each
  FillSlice fill;        // done by extra workgroups of the column pass
  int cw = 1;
  // forward only (else null): per preparation workgroup, kPresWords words of
  // presence bits of its GT labels, [B][nblk][kPresWords]; every word is
  // rewritten on each call, so nothing needs clearing first
  uint32_t* pbits = nullptr;
  int nblk = 0;          // preparation workgroups per image (prep_blocks)
  // void-class check (reference functions/mask/matching.py:184-185): an extra
  // workgroup of the preparation launch (blockIdx.x == nblk, image 0) writes
  // *void_found = any(cls_targets == void_idx) (device or host-mapped memory)
  const int64_t* cls_targets = nullptr;
  int64_t void_idx = -1;  // -1: no valid void index (the check reports 0)
  int32_t* void_found = nullptr;
  // null, or kClasses int32 the device can write (pinned host memory mapped
  // for the device): the column pass stores each class's task count there
  // with system-scope stores, for a host that launches only non-empty classes
  int32_t* class_counts = nullptr;
  // the assignment's finished-image count (see AssignArgs::done), zeroed by
  // the column pass, or null
  int* done = nullptr;
  int* ncols;
  int* colmap;
  int* slot_of_col;
  int* sched;            // cost schedule (see CostPlan), or null
  int64_t B, H, W, Ht, Wt, s, HWp, GT_total, GT_out, bg;
  int nslot;
  int64_t L, rtiles;
  CostPlan plan;
};

struct CostArgs {
  const void* logits;
  const uint16_t* lab16;
  const uint8_t* counts;  // s > 1: [B][GT_total][HWp] counts of cw bytes each
  int cw;
  const int* ncols;
  const int* colmap;
  const int* sched;  // device schedule (see CostPlan)
  float* partials;   // per work item: [planes][rows][16 * NT_class] (CostPlan::planes)
  float* rowsum;     // per work item: [rows][2] unweighted (force_masks) or null
  CostPlan plan;
  int64_t L, B, Q, HW, HWp, rtiles, GT_total, bg, rows;
  int nslot;
  float N2;
  ElemParams ep;
  int use_lut;       // bf16 logits: per-cell planes from the LDS table
};

struct LayerArgs {
  const float* img;
  float* layer;        // [L][ML_LAYERS]
  float* means;        // (3, L)
  const int64_t* pred_to_gt;
  int* list;           // matched-row list of the saved state, or null
  int* mrows;          // [L*B][Q]: slice lb's matched rows (lb * Q + q, ascending), its
                       // count in img[lb * 4 + 3]; written by the assignment when list is set
  int64_t L, B, Q;
  double num_masks;
  int force_masks, force_cls, has_void;
};

struct AssignArgs {
  // inputs
  const void* cls_logits;
  int cls_dtype;
  const int64_t* cls_targets;
  const float* partials;
  const float* rowsum;
  const int* sched;
  CostPlan plan;
  const int* ncols;
  const int* slot_of_col;
  const int* colmap;     // [B][nslot]: output column of each non-empty GT slot
  // outputs
  float* sep;            // (3, L, B, Q, GT_out): bce, dice, label cost
  float* out_bce;        // where finalize writes the bce / dice planes (sep's
  float* out_dice;       // first two planes, or a standalone operator's outputs, or null)
  float* tot;            // [LB][tot_stride] total cost (bce + dice) + label, [c][q], or null
  int64_t tot_stride;    // Q * GT_out rounded up to whole 16-byte words
  // [LB][GT_out][Q] float64 copies of the staged cost rows with the invalid
  // cost replaced by `big` (the Hungarian's c(i, j)), written by the
  // assignment's staging pass when the rows are read in place (they do not
  // fit the LDS), or null
  double* tot64 = nullptr;
  float* rowIT;          // [LB*Q][nslot][2] summed I, T per column slot, or null
  int64_t* pred_to_gt;   // (L,B,Q) or null (costs-only mode)
  int64_t* pred_round;
  float* stats;          // (L,B,Q,ML_STATS) or null
  float* rowstat;        // [LB*Q][8]: S, P, mask pen, dice pen, cls pen
  float* img;            // [LB][4]: mask, dice, cls sums, matched count
  // gradient zero-fill done by extra workgroups of the assignment launch
  // (blockIdx.x >= L*B), or fill_blocks == 0
  FillSlice fin_fill;  // done by extra workgroups of the finalize launch
  u32x4_t* fill;
  int64_t fill_n16;
  unsigned char* fill_tail;
  int64_t fill_ntail;
  int fill_blocks;
  // finished-image count (zeroed by finalize when reset_done is set, else
  // by the column pass): the assignment workgroup that finishes last runs
  // the per-layer pass `layer_args`, or done == null
  int* done;
  int reset_done = 1;
  // image subset of this finalize / assignment launch: every image when
  // phase_class < 0, else the images whose column-tile class (class_of(G +
  // 1)) is phase_class (phase_in = 1) or is not (phase_in = 0).  Each row's
  // and image's work is its own, so two complementary launches give the
  // results of one launch over every image.
  int phase_class = -1;
  int phase_in = 1;
  LayerArgs layer_args;
  // dims / params
  int64_t L, B, Q, C, HW, Ht, Wt, GT_total, GT_out, bg, rtiles;
  int rows, nslot;
  float N2;
  float smooth, sigmoid_scale, dice_scale, cls_scale;
  int normalize, use_softmax, force_cls, force_masks;
  int64_t void_idx;
  float cls_gamma, cls_alpha;
  ElemParams cls_ep;
  ElemParams mask_ep;
  double inf_thresh, big;
  int64_t topk;
  int strategy;
  int costs_only;
  int64_t lds_rows;  // GT_out when the assignment keeps every cost row in LDS, else 0
};


struct BwdArgs {
  const void* logits;
  int dtype;
  const uint16_t* lab16;
  const uint8_t* counts;  // s > 1: [B][GT_total][HWp] counts of cw bytes each
  int cw;
  const int64_t* pred_to_gt;
  const float* stats;     // per-query stats or null
  const int* list;        // matched-row list (count, rows): only these rows are written
  const float* layer;     // [L][ML_LAYERS]
  const float* g_mask;
  const float* g_dice;
  const float* g_cls;
  void* grad;             // (L,B,Q,HW) in dtype
  const void* cls_logits;
  int cls_dtype;
  const int64_t* cls_targets;
  void* grad_cls;
  int64_t L, B, Q, HW, HWp, C, GT_total, bg, Ht, Wt;
  float N2;
  float smooth, sigmoid_scale, dice_scale, cls_scale;
  int normalize, force_masks, force_cls, use_softmax;
  int64_t void_idx;
  ElemParams mask_ep;
  ElemParams cls_ep;
  float cls_gamma;
  int cls_fused;          // the mask kernel also writes the class-logit gradients
};

// Non-pairwise sigmoid-CE / dice over dense class logits (L, B, C, H, W).
struct DenseArgs {
  const void* logits;
  int dtype;
  const uint16_t* lab16;   // s == 1: label per cell (0xFFFF outside [0, C))
  const uint8_t* counts;   // s > 1: [B][C][HWp] per-cell counts of cw bytes each
  int cw;
  int64_t L, B, C, HW, HWp, HtWt;
  float N2;
  ElemParams ep;           // focal terms (sigmoid CE)
  float scale, smooth;
  double num_masks;
  double* partials;        // forward: per (plane, chunk) float64 sums
  float* loss;             // (L,)
  float *I_out, *P_out, *T_out;                // dice forward: (L, B, C)
  const float* grad_out;                       // backward: (L,)
  const float *I_in, *P_in, *T_in;             // dice backward
  void* grad;                                  // (L, B, C, H, W) in dtype
};

// ---- the shared forward (ml_capi.hip) ---------------------------------------
// prep -> cost -> finalize -> assignment (costs_only: no assignment) on `st`,
// scratch from `ws` (ws_bytes).  packed: the cost plan's regions are packed
// for its own slot counts (pack_cost_plan) instead of the kCostSlots bound,
// with fewer slots where that does not fit ws_bytes (fit_cost_plan).
// cc_dev / cc_host: null, or the device and host addresses of kClasses pinned
// int32 words: the column pass stores the classes' task counts there, and the
// host launches one class (class 0 of two, the widest of three), waits for
// the counts, then launches only the other classes that have tasks.
int forward_impl(const ml_shape* s, const ml_params* p, int mask_dtype, const void* mask_logits,
                 const int64_t* mask_targets, int cls_dtype, const void* cls_logits,
                 const int64_t* cls_targets, int64_t* pred_to_gt, int64_t* pred_round,
                 float* layer_means, float* sep, void* saved, void* prefill, int32_t* void_found,
                 hipEvent_t void_ready, void* ws, size_t ws_bytes, hipStream_t st, bool costs_only,
                 float* bce_out, float* dice_out, const float* pt_coords, int64_t pt_Hs,
                 int64_t pt_Ws, bool packed, int32_t* cc_dev = nullptr,
                 volatile int32_t* cc_host = nullptr);
// Workspace bytes of the packed forward whose cost plan is fitted to `budget`
// (fit_cost_plan), what forward_impl with packed = true and ws_bytes = budget
// uses.
int forward_packed_bytes(const ml_shape* s, const ml_params* p, int mask_dtype, size_t budget,
                         size_t& bytes);
int check_matching_params(const ml_params* p, int64_t C);

// ---- instrumentation: bracket a launch with events when profiling is on ------
void prof_begin(const char* name, hipStream_t st);
void prof_end(const char* name, hipStream_t st);
struct ProfScope {
  const char* n;
  hipStream_t s;
  // name == null: no bracket
  ProfScope(const char* name, hipStream_t st) : n(name), s(st) {
    if (n) prof_begin(n, s);
  }
  ~ProfScope() {
    if (n) prof_end(n, s);
  }
};

// ---- launchers (defined in the kernels' translation units) ---------------------
int launch_prep(const PrepArgs& a, const Dims& d, hipStream_t st);
// classes: bit c launches column-tile class c (all by default); prof: bracket
// the launches with the profiling events
int launch_cost(const CostArgs& a, const Dims& d, int dtype, bool force_masks, hipStream_t st,
                unsigned classes = ~0u, bool prof = true);
int launch_finalize(const AssignArgs& a, const Dims& d, hipStream_t st,
                    const char* prof = "finalize");
int launch_assign(const AssignArgs& a, const Dims& d, hipStream_t st, const char* prof = "assign");
int launch_layer(const LayerArgs& a, hipStream_t st);
int launch_layer_from_p2g(const int64_t* p2g, float* layer, int64_t L, int64_t B, int64_t Q,
                          double num_masks, int force_masks, int force_cls, int has_void,
                          hipStream_t st);
int launch_bwd(const BwdArgs& a, const Dims& d, hipStream_t st);
int launch_label_cost(const void* cls_logits, int cls_dtype, const int64_t* cls_targets,
                      int64_t L, int64_t B, int64_t Q, int64_t C, int64_t GT_total,
                      int64_t GT_out, int64_t bg, float scale, const ElemParams& ep,
                      int use_softmax, float* out, hipStream_t st);
int launch_fill_i32(int* p, int v, int64_t n, hipStream_t st);
int prep_blocks(const Dims& d);
// point-sampling front end (ml_points.hip, ml_prep.hip)
int prep_blocks_map(int64_t Hs, int64_t Ws);
int launch_prep_points(const PrepArgs& a, const Dims& d, int64_t Hs, int64_t Ws, const float* coords,
                       hipStream_t st);
int launch_point_sample(int dtype, const void* in, const float* coords, int64_t N, int64_t C,
                        int64_t H, int64_t W, int64_t P, int64_t cb, int align, void* out,
                        hipStream_t st);
size_t point_sample_bwd_workspace(int dtype, int64_t N, int64_t C, int64_t H, int64_t W, int64_t P,
                                  int64_t cb);
int launch_point_sample_backward(int dtype, const void* gout, const float* coords, int64_t N,
                                 int64_t C, int64_t H, int64_t W, int64_t P, int64_t cb, int align,
                                 void* gin, float* acc, hipStream_t st);
int launch_point_labels(const int64_t* targets, const float* coords, int64_t B, int64_t Ht,
                        int64_t Wt, int64_t P, int64_t GT_total, int64_t* out64, uint16_t* out16,
                        int64_t HWp, hipStream_t st);
int launch_dense(const DenseArgs& a, bool dice, bool backward, hipStream_t st);
size_t dense_partials_bytes(int64_t L, int64_t B, int64_t C, int64_t HW, bool dice);
int launch_zero_fill(void* p, size_t bytes, hipStream_t st);

// Zero `n16` 16-byte words, then `ntail` trailing bytes, as workgroup `blk`
// of `nblk` (of equal size).  Streaming (non-temporal) stores: the buffer
// is a gradient that is not read again before the backward, so it should not
// displace the forward's working set from the L2.
__device__ inline void zero_fill_range(u32x4_t* p, int64_t n16, unsigned char* tail,
                                       int64_t ntail, int64_t blk, int64_t nblk) {
  const int64_t nt = blockDim.x, stride = nblk * nt;
  int64_t i = blk * nt + threadIdx.x;
  const u32x4_t z = {0u, 0u, 0u, 0u};
  for (; i + 3 * stride < n16; i += 4 * stride) {
    __builtin_nontemporal_store(z, p + i);
    __builtin_nontemporal_store(z, p + i + stride);
    __builtin_nontemporal_store(z, p + i + 2 * stride);
    __builtin_nontemporal_store(z, p + i + 3 * stride);
  }
  for (; i < n16; i += stride) __builtin_nontemporal_store(z, p + i);
  if (blk == 0 && threadIdx.x < ntail) tail[threadIdx.x] = 0;
}
__device__ inline void fill_slice(const FillSlice& f, int64_t blk) {
  zero_fill_range(f.p, f.n16, nullptr, 0, blk, f.blocks);
}
int launch_any_equal(const int64_t* x, int64_t n, int64_t value, int32_t* flag, hipStream_t st);
int launch_stream_read(const void* p, int64_t n16, uint32_t* out, int grid, hipStream_t st);

// Counts of one label at 8 consecutive cells starting at element `idx` of the
// count tensor: u8 (cw == 1) or u16 (cw == 2).  idx is a multiple of 8, so the
// run is one aligned 8- or 16-byte load.  The reference's uint8 counts
// (src/cuda/utils.cuh:9) overflow for s >= 16; u16 holds up to s = 255.
__device__ __forceinline__ void counts8_u32(const uint8_t* base, int cw, int64_t idx, uint32_t n[8]) {
  if (cw == 1) {
    const uint2 v = *(const uint2*)(base + idx);
    const uint32_t w[2] = {v.x, v.y};
#pragma unroll
    for (int k = 0; k < 8; ++k) n[k] = (w[k >> 2] >> ((k & 3) * 8)) & 0xFFu;
  } else {
    const uint4 v = *(const uint4*)(base + 2 * idx);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 8; ++k) n[k] = (w[k >> 1] >> ((k & 1) * 16)) & 0xFFFFu;
  }
}
__device__ __forceinline__ void counts8_f(const uint8_t* base, int cw, int64_t idx, float n[8]) {
  uint32_t u[8];
  counts8_u32(base, cw, idx, u);
#pragma unroll
  for (int k = 0; k < 8; ++k) n[k] = (float)u[k];
}

}  // namespace ml
