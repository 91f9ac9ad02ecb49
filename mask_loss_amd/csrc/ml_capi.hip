// C ABI entry points (declared in include/mask_loss_hip.h): argument
// validation mirroring the reference's checks, workspace layout and the
// launch sequence of each operator.  Host code only; all work is enqueued on
// the caller's stream.
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "ml_internal.h"

namespace ml {

static thread_local std::string g_err;
int g_use_lut = 1;  // bf16 per-cell planes from the LDS table (0: formulas, for tests)

void set_error(const std::string& msg) { g_err = msg; }
int fail(int code, const std::string& msg) {
  set_error(msg);
  return code;
}
int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(ML_ELAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  return ML_OK;
}

size_t assign_smem_bytes(int64_t Q, int64_t GTo, int64_t lds_rows);

// ---- instrumentation ----------------------------------------------------------
namespace {
struct ProfRec {
  const char* name;
  hipEvent_t a, b;
};
std::mutex g_prof_mu;
bool g_prof_on = false;
std::vector<hipEvent_t> g_pool;
std::vector<ProfRec> g_recs;
std::vector<std::pair<const char*, hipEvent_t>> g_open;

hipEvent_t take_event() {
  if (g_pool.empty()) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }
  hipEvent_t e = g_pool.back();
  g_pool.pop_back();
  return e;
}
}  // namespace

void prof_begin(const char* name, hipStream_t st) {
  if (!g_prof_on) return;
  std::lock_guard<std::mutex> g(g_prof_mu);
  hipEvent_t e = take_event();
  if (!e) return;
  (void)hipEventRecord(e, st);
  g_open.push_back({name, e});
}

void prof_end(const char* name, hipStream_t st) {
  if (!g_prof_on) return;
  std::lock_guard<std::mutex> g(g_prof_mu);
  for (size_t i = g_open.size(); i-- > 0;) {
    if (strcmp(g_open[i].first, name) == 0) {
      hipEvent_t e = take_event();
      if (!e) return;
      (void)hipEventRecord(e, st);
      g_recs.push_back({name, g_open[i].second, e});
      g_open.erase(g_open.begin() + (long)i);
      return;
    }
  }
}


constexpr size_t kMaxLds = 160 * 1024;

bool make_dims(const ml_shape* s, int64_t background_index, int dtype, Dims& d,
               std::string& err) {
  d.L = s->L; d.B = s->B; d.Q = s->Q; d.H = s->H; d.W = s->W;
  d.Ht = s->Ht; d.Wt = s->Wt; d.C = s->C; d.GT_total = s->GT_total;
  if (d.L < 0 || d.B < 0 || d.Q < 0 || d.C < 0 || d.GT_total < 0) {
    err = "negative dimension";
    return false;
  }
  if (d.H <= 0 || d.W <= 0) {
    err = "mask_logits must have positive spatial size";
    return false;
  }
  if (d.Ht % d.H != 0 || d.Wt % d.W != 0 || d.Ht / d.H != d.Wt / d.W || d.Ht == 0) {
    err = "Target resolution must be the same integer multiple of the mask_logits resolution in both dimensions";
    return false;
  }
  d.s = d.Ht / d.H;
  if (d.s > 255) {
    err = "target/logit scale factors above 255 are not supported (per-cell counts are 16-bit)";
    return false;
  }
  if (d.GT_total > 65535) {
    err = "at most 65535 GT slots per image are supported";
    return false;
  }
  d.N2 = d.s * d.s;
  d.LB = d.L * d.B;
  d.HW = d.H * d.W;
  const bool skip = background_index >= 0 && background_index < d.GT_total;
  d.bg = background_index >= 0 ? background_index : d.GT_total;
  d.GT_out = d.GT_total - (skip ? 1 : 0);
  d.HWp = ceil_div(d.HW, kStep) * kStep;
  const int64_t need = ceil_div(d.GT_out + 1, 16);  // + ones column
  if (need <= 2) d.NT = 2;
  else if (need <= 7) d.NT = 7;
  else if (need <= 16) d.NT = 16;
  else {
    err = "more than 255 GT columns per image are not supported";
    return false;
  }
  d.RT = cost_rt_for(dtype, d.NT);
  d.rows = 16 * d.RT;
  d.nslot = 16 * d.NT;
  d.rtiles = ceil_div(d.Q, d.rows);
  // a wave covers at least 4 K-steps of its task (small maps then split
  // further and fill more of the GPU: a 64 x 64 map with 14 row tiles takes
  // 15.8 us instead of 24.5 with 8; large maps are bound by the resident
  // slots, not by this)
  const int64_t nsteps = ceil_div(d.HW, kStep);
  d.ks_max = nsteps / 4 > 1 ? nsteps / 4 : 1;
  d.counts_mode = d.s > 1;
  d.cw = d.s >= 16 ? 2 : 1;  // u8 counts overflow at s*s >= 256
  // row-tile pairs stream 16-byte aligned rows (HW % 8 == 0) with 32-bit
  // element offsets within a pair's 32 rows
  d.pair_ok = dtype == ML_BF16 && !d.counts_mode && d.rows == 16 && d.HW % 8 == 0 && d.HW >= 8 &&
              d.HW * 32 < ((int64_t)1 << 31);
  return true;
}

// Class regions sized for max(kCostSlots, tasks) work items each; slots are
// the workspace bound (kCostSlots).
CostPlan bound_cost_plan(const Dims& d) {
  CostPlan p{};
  p.ntasks = d.LB * d.rtiles;
  p.rtiles = d.rtiles;
  p.ks_max = d.ks_max;
  p.pair0 = 0;
  p.nclass = 0;
  while (p.nclass < kClasses && class_nt(p.nclass) <= d.NT) ++p.nclass;
  const int64_t cap = std::max<int64_t>(kCostSlots, p.ntasks);
  int64_t f = 0;
  for (int c = 0; c < kClasses; ++c) {
    p.slots[c] = (int)kCostSlots;
    p.slot_base[c] = (int64_t)c * cap;
    p.float_base[c] = f;
    // row-tile pairs: up to max(slots, pairs) items of two row tiles each
    const int64_t items = c == 0 && d.pair_ok ? 2 * cap : cap;
    p.planes[c] = c == 0 ? 3 : 4;  // the most any plan of this shape uses
    if (c < p.nclass) f += items * p.planes[c] * d.rows * 16 * class_nt(c);
  }
  p.float_total = f;
  p.slot_total = (int64_t)p.nclass * cap;
  return p;
}

void pack_cost_plan(CostPlan& p, const Dims& d) {
  int64_t f = 0, sl = 0;
  for (int c = 0; c < kClasses; ++c) {
    const int64_t cap = c < p.nclass ? std::max<int64_t>(p.slots[c], p.ntasks) : 0;
    p.slot_base[c] = sl;
    p.float_base[c] = f;
    sl += cap;
    f += (c == 0 && p.pair0 ? 2 * cap : cap) * p.planes[c] * d.rows * 16 * class_nt(c);
  }
  p.float_total = f;
  p.slot_total = sl;
}

// The packed plan within `budget` workspace bytes: while the layout exceeds
// it, halve the slots of the class whose partial-sum region is largest (a
// smaller K-split and grid for that class: slower, same results to the cost
// tolerance), down to the class's task count.  For the allocation-free
// forward, whose scratch is fixed.
void fit_cost_plan(CostPlan& p, const Dims& d, bool force_masks, size_t budget) {
  pack_cost_plan(p, d);
  while (make_layout(d, force_masks, p).total > budget) {
    int best = -1;
    int64_t best_f = 0;
    for (int c = 0; c < p.nclass; ++c) {
      const int64_t f = (c + 1 < kClasses ? p.float_base[c + 1] : p.float_total) - p.float_base[c];
      if (p.slots[c] > 8 && p.slots[c] > p.ntasks && f > best_f) {
        best = c;
        best_f = f;
      }
    }
    if (best < 0) return;
    p.slots[best] = std::max<int>(8, p.slots[best] / 2);
    pack_cost_plan(p, d);
  }
}

static int64_t cost_lds_rows(const Dims& d);

Layout make_layout(const Dims& d, bool force_masks) {
  return make_layout(d, force_masks, bound_cost_plan(d));
}

Layout make_layout(const Dims& d, bool force_masks, const CostPlan& pl) {
  Layout L;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t r = o;
    o = align256(o + bytes);
    return r;
  };
  L.lab16 = take(d.counts_mode ? 0 : (size_t)d.B * d.HWp * 2);
  L.counts = take(d.counts_mode ? (size_t)d.B * d.GT_total * d.HWp * d.cw : 0);
  L.pbits = take((size_t)d.B * prep_blocks(d) * kPresWords * 4);
  L.ncols = take((size_t)d.B * 4);
  L.colmap = take((size_t)d.B * d.nslot * 4);
  L.slot_of_col = take((size_t)d.B * d.GT_out * 4);
  L.sched = take((size_t)sched_ints(pl.ntasks) * 4);
  L.partials = take((size_t)pl.float_total * 4);
  L.rowsum = take(force_masks ? (size_t)pl.slot_total * d.rows * 2 * 4 : 0);
  L.sep = take((size_t)3 * d.LB * d.Q * d.GT_out * 4);
  L.tot = take((size_t)d.LB * ceil_div(d.Q * d.GT_out, 4) * 16);
  // float64 cost rows for an assignment that reads them in place
  L.tot64 = take(cost_lds_rows(d) == 0 ? (size_t)d.LB * d.GT_out * d.Q * 8 : 0);
  L.rowIT = take((size_t)d.LB * d.Q * d.nslot * 8);
  L.rowstat = take((size_t)d.LB * d.Q * 8 * 4);
  L.img = take((size_t)d.LB * 4 * 4);
  L.mrows = take((size_t)d.LB * d.Q * 4);
  L.layer = take((size_t)d.L * ML_LAYERS * 4);
  L.done = take(16);
  L.total = o;
  return L;
}

// Shapes the assignment launch supports, checked before anything is queued:
// one wave holds a cost row of at most 1024 queries in registers (16 per
// lane), and the workgroup's per-query arrays must fit the LDS without any
// cost row.
static bool check_assign_dims(const Dims& d, std::string& err) {
  if (d.Q > 1024) {
    err = "more than 1024 queries per image are not supported by the assignment";
    return false;
  }
  if (assign_smem_bytes(d.Q, d.GT_out, 0) > kMaxLds - 1024) {
    err = "assign: the per-query arrays exceed the LDS budget";
    return false;
  }
  return true;
}

// Cost rows (by column) the assignment keeps in LDS: all GT_out of them when
// they fit, else none (every row is then read in place from L2: on the
// widest images that beats keeping only the first rows in LDS, whose staging
// writes cost more than the L2 reads they replace, since each Dijkstra step
// is bound by its own instruction chain and not by the row read).
// 1 KB stays free for the assignment kernel's static LDS.
static int64_t cost_lds_rows(const Dims& d) {
  return assign_smem_bytes(d.Q, d.GT_out, d.GT_out) <= kMaxLds - 1024 ? d.GT_out : 0;
}

// The matching forward's required device pointers: every input and the three
// outputs (a shape with no query rows reads and writes none of them).
static int check_matching_pointers(const ml_shape* s, const void* mask_logits,
                                   const int64_t* mask_targets, const void* cls_logits,
                                   const int64_t* cls_targets, const int64_t* pred_to_gt,
                                   const int64_t* pred_round, const float* layer_means) {
  if (s->L <= 0 || s->B <= 0 || s->Q <= 0) return ML_OK;
  if (!mask_logits || !mask_targets || !cls_logits || !cls_targets || !pred_to_gt || !pred_round ||
      !layer_means)
    return fail(ML_EINVAL, "matching forward: a required input or output pointer is null");
  return ML_OK;
}

static int check_focal(float gamma, float alpha, const char* who) {
  if (!(gamma >= 0.f)) return fail(ML_EINVAL, std::string(who) + " focal_gamma must be non-negative");
  if (!(alpha < 0.f || (alpha >= 0.f && alpha <= 1.f)))
    return fail(ML_EINVAL, std::string(who) + " focal_alpha must be in [0, 1] or negative to disable");
  return ML_OK;
}

static int check_params(const ml_params* p, int64_t C, bool matching) {
  int rc;
  if ((rc = check_focal(p->mask_gamma, p->mask_alpha, "mask"))) return rc;
  if ((rc = check_focal(p->cls_gamma, p->cls_alpha, "cls"))) return rc;
  if (matching) {
    if (p->topk_matches < 0) return fail(ML_EINVAL, "K must be non-negative");
    if (p->strategy_id < 0 || p->strategy_id > 3) return fail(ML_EINVAL, "Invalid matching strategy id");
    if (!(p->uncertainty_gamma >= 0.f))
      return fail(ML_EINVAL, "uncertainty_gamma must be non-negative");
    if (!(p->uncertainty_gamma_min >= 0.f && p->uncertainty_gamma_min <= 1.f))
      return fail(ML_EINVAL, "uncertainty_gamma_min must be in [0,1]");
    if (p->use_softmax_label_loss && p->force_unmatched_class_to_background &&
        !(p->void_class_index >= 0 && p->void_class_index < C))
      return fail(ML_EINVAL,
                  "void_class_index must be provided when using softmax label loss and forcing "
                  "unmatched class logits");
  }
  return ML_OK;
}

int check_matching_params(const ml_params* p, int64_t C) { return check_params(p, C, true); }

static bool dtype_ok(int dt) { return dt == ML_F32 || dt == ML_BF16 || dt == ML_F16; }

// The task counts of the column-tile classes below nclass other than `skip`
// from the pinned words the column pass stores with system scope (preset to
// -1): polled, and after 2 s the stream is drained, after which they are
// written.
static int wait_class_counts(volatile int32_t* w, int nclass, int skip, hipStream_t st, int32_t* n) {
  const auto t0 = std::chrono::steady_clock::now();
  auto ready = [&]() {
    for (int c = 0; c < nclass; ++c)
      if (c != skip && w[c] == -1) return false;
    return true;
  };
  while (!ready()) {
    if (std::chrono::steady_clock::now() - t0 > std::chrono::seconds(2)) {
      if (hipStreamSynchronize(st) != hipSuccess) return fail(ML_ELAUNCH, "class counts: stream failed");
      if (!ready()) return fail(ML_ELAUNCH, "class counts: the column pass did not write them");
      break;
    }
    std::this_thread::yield();
  }
  for (int c = 0; c < kClasses; ++c) n[c] = c < nclass && c != skip ? w[c] : 0;
  return ML_OK;
}

// A second stream of the current device with a fork and a join event, taken
// from a pool for the span of one forward's enqueueing.  The stream has the
// default priority and does not synchronise with the null stream; an event
// may be recorded again once the wait on it is enqueued, so an entry goes
// back to the pool right after the join wait.
struct SideStream {
  int dev = -1;
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
static std::mutex g_side_mu;
static std::vector<SideStream> g_side_free;

static int side_acquire(SideStream& out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(ML_ELAUNCH, "no current device");
  {
    std::lock_guard<std::mutex> g(g_side_mu);
    for (size_t i = 0; i < g_side_free.size(); ++i)
      if (g_side_free[i].dev == dev) {
        out = g_side_free[i];
        g_side_free.erase(g_side_free.begin() + (long)i);
        return ML_OK;
      }
  }
  SideStream n;
  n.dev = dev;
  if (hipStreamCreateWithFlags(&n.s, hipStreamNonBlocking) != hipSuccess)
    return fail(ML_ELAUNCH, "cannot create the side stream");
  if (hipEventCreateWithFlags(&n.fork, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&n.join, hipEventDisableTiming) != hipSuccess) {
    if (n.fork) (void)hipEventDestroy(n.fork);
    (void)hipStreamDestroy(n.s);
    return fail(ML_ELAUNCH, "cannot create the side stream's events");
  }
  out = n;
  return ML_OK;
}
static void side_release(const SideStream& ss) {
  std::lock_guard<std::mutex> g(g_side_mu);
  g_side_free.push_back(ss);
}

// Shared forward: prep -> cost -> assign (-> layer).
int forward_impl(const ml_shape* s, const ml_params* p, int mask_dtype,
                 const void* mask_logits, const int64_t* mask_targets, int cls_dtype,
                 const void* cls_logits, const int64_t* cls_targets, int64_t* pred_to_gt,
                 int64_t* pred_round, float* layer_means, float* sep, void* saved,
                 void* prefill, int32_t* void_found, hipEvent_t void_ready, void* ws,
                 size_t ws_bytes, hipStream_t st, bool costs_only, float* bce_out,
                 float* dice_out, const float* pt_coords, int64_t pt_Hs, int64_t pt_Ws,
                 bool packed, int32_t* cc_dev, volatile int32_t* cc_host) {
  if (!dtype_ok(mask_dtype) || (cls_logits && !dtype_ok(cls_dtype)))
    return fail(ML_EINVAL, "unsupported dtype");
  Dims d;
  std::string err;
  if (!make_dims(s, p->background_index, mask_dtype, d, err)) return fail(ML_EINVAL, err);
  if (!costs_only && !check_assign_dims(d, err)) return fail(ML_EUNSUPPORTED, err);
  if (!costs_only) {
    const int rc = check_matching_pointers(s, mask_logits, mask_targets, cls_logits, cls_targets,
                                           pred_to_gt, pred_round, layer_means);
    if (rc) return rc;
  }
  const bool force_masks = !costs_only && p->force_unmatched_masks_to_empty;
  if (prefill && (force_masks || costs_only || !saved))
    return fail(ML_EINVAL, "gradient prefill needs a saved state and unforced unmatched masks");
  if (((uintptr_t)prefill & 15) || ((uintptr_t)saved & 255))
    return fail(ML_EINVAL, "the prefill buffer must be 16-byte and the saved state 256-byte aligned");
  const int64_t lds_rows = cost_lds_rows(d);
  const SavedLayout SL = saved_layout(d);
  unsigned char* sv = (unsigned char*)saved;
  float* stats = saved ? (float*)(sv + SL.stats) : nullptr;
  const bool tab = mask_dtype == ML_BF16 && !d.counts_mode && g_use_lut && !force_masks;
  CostPlan plan = make_cost_plan(d, mask_dtype, tab);
  if (packed) fit_cost_plan(plan, d, force_masks, ws_bytes);
  const Layout L = packed ? make_layout(d, force_masks, plan) : make_layout(d, force_masks);
  // point-sampling front end: presence records of the full label map after the layout
  const size_t pt_pbits = align256(L.total);
  const int pt_nblk = pt_coords ? prep_blocks_map(pt_Hs, pt_Ws) : 0;
  const size_t need = pt_coords ? pt_pbits + (size_t)d.B * pt_nblk * kPresWords * 4 : L.total;
  if (ws_bytes < need) return fail(ML_EWORKSPACE, "workspace too small");
  unsigned char* w = (unsigned char*)ws;
  int rc;
  // the gradient's zero fill (16-byte words): slices for the column pass and
  // the finalize launch, the rest (and any tail bytes) for the assignment
  // launch, or one fill kernel without an assignment launch
  const size_t prefill_bytes =
      prefill && !costs_only ? (size_t)(d.LB * d.Q * d.HW) * (mask_dtype == ML_F32 ? 4 : 2) : 0;
  const int64_t fill_n16 = (int64_t)(prefill_bytes / 16);
  auto slice = [&](int64_t from, int64_t cap) {
    FillSlice f;
    f.n16 = d.LB > 0 ? std::max<int64_t>(0, std::min<int64_t>(fill_n16 - from, cap / 16)) : 0;
    f.p = f.n16 ? (u32x4_t*)prefill + from : nullptr;
    f.blocks = f.n16 ? (int)std::min<int64_t>(kFillBlocks, ceil_div(f.n16, 1024)) : 0;
    return f;
  };
  // with three column-tile classes the polled forward may split the images
  // (the widest class's assignment on a side stream, the critical path): the
  // column pass, which that path waits for, then leaves its share to the
  // other images' assignment launch
  const FillSlice prep_fill = slice(0, plan.nclass == kClasses ? 0 : kPrepFillBytes);
  const FillSlice fin_fill = slice(prep_fill.n16, kFinFillBytes);
  const int64_t assign_from = prep_fill.n16 + fin_fill.n16;

  PrepArgs pa;
  pa.fill = prep_fill;
  pa.targets = mask_targets;
  // with a saved state the compact labels go straight into it (the backward reuses them)
  pa.lab16 = (uint16_t*)(saved && !d.counts_mode ? sv + SL.lab16 : w + L.lab16);
  pa.counts = (uint8_t*)(w + L.counts);
  pa.cw = d.cw;
  pa.pbits = (uint32_t*)(w + L.pbits);
  pa.nblk = prep_blocks(d);
  const int64_t void_idx =
      (p->void_class_index >= 0 && p->void_class_index < d.C) ? p->void_class_index : -1;
  if (void_found) {
    pa.cls_targets = cls_targets;
    pa.void_idx = cls_targets ? void_idx : -1;
    pa.void_found = void_found;
  }
  pa.ncols = (int*)(w + L.ncols);
  pa.colmap = (int*)(w + L.colmap);
  pa.slot_of_col = (int*)(w + L.slot_of_col);
  pa.B = d.B; pa.H = d.H; pa.W = d.W; pa.Ht = d.Ht; pa.Wt = d.Wt; pa.s = d.s; pa.HWp = d.HWp;
  pa.GT_total = d.GT_total; pa.GT_out = d.GT_out; pa.bg = d.bg; pa.nslot = d.nslot;
  pa.sched = (int*)(w + L.sched);
  pa.done = costs_only ? nullptr : (int*)(w + L.done);
  pa.L = d.L; pa.rtiles = d.rtiles; pa.plan = plan;
  // the wider classes' launches wait for the device's task counts (only when
  // there are wider classes and a host that can wait)
  const bool poll_classes = cc_dev && cc_host && !pt_coords && plan.nclass > 1;
  if (poll_classes) {
    for (int c = 0; c < kClasses; ++c) cc_host[c] = -1;
    pa.class_counts = cc_dev;
  }
  if (pt_coords) {
    pa.pbits = (uint32_t*)(w + pt_pbits);
    pa.nblk = pt_nblk;
    if (d.B > 0 && (rc = launch_prep_points(pa, d, pt_Hs, pt_Ws, pt_coords, st))) return rc;
  } else if (d.B > 0 && (rc = launch_prep(pa, d, st))) {
    return rc;
  }
  if (void_found && d.B == 0 && (rc = launch_fill_i32(void_found, 0, 1, st))) return rc;
  if (void_ready && hipEventRecord(void_ready, st) != hipSuccess)
    return fail(ML_ELAUNCH, "cannot record the void-check event");

  const ElemParams mask_ep = make_elem_params(p->mask_gamma, p->mask_alpha,
                                              p->uncertainty_gamma, p->uncertainty_gamma_min);
  CostArgs ca;
  ca.logits = mask_logits;
  ca.lab16 = pa.lab16;
  ca.counts = d.counts_mode ? pa.counts : nullptr;
  ca.cw = d.cw;
  ca.ncols = pa.ncols;
  ca.colmap = pa.colmap;
  ca.sched = pa.sched;
  ca.plan = plan;
  ca.partials = (float*)(w + L.partials);
  ca.rowsum = force_masks ? (float*)(w + L.rowsum) : nullptr;
  ca.L = d.L; ca.B = d.B; ca.Q = d.Q; ca.HW = d.HW; ca.HWp = d.HWp;
  ca.rtiles = d.rtiles; ca.GT_total = d.GT_total; ca.bg = d.bg; ca.rows = d.rows;
  ca.nslot = d.nslot; ca.N2 = (float)d.N2; ca.ep = mask_ep;
  ca.use_lut = g_use_lut;
  // Two image subsets when the widest class (more than 111 non-empty GTs:
  // the longest solver chains) is the first and the polled counts show
  // another non-empty class: the widest class's finalize runs right after
  // its contraction and its assignment on a side stream, beside the other
  // classes' contraction, finalize and assignment here.  The other classes'
  // launches leave kSideCUs CUs free for it (CostPlan::slots), and each
  // subset's rows and images are computed exactly as in one launch, so the
  // results are the same.
  int phase_first = -1;
  unsigned rest_classes = 0;
  SideStream side;
  if (d.LB > 0 && d.rtiles > 0) {
    if (!poll_classes) {
      if ((rc = launch_cost(ca, d, mask_dtype, force_masks, st))) return rc;
    } else {
      // one class first, unconditionally: class 0 when the shape allows two
      // classes, else the widest; while it runs, the column pass's counts
      // reach the host, which then launches only the other classes that have
      // tasks (an empty class launch costs the GPU ~4.5 us, and waiting
      // before the first class would leave the GPU idle instead)
      ProfScope ps_("pair_cost", st);
      const int first = plan.nclass > 2 ? plan.nclass - 1 : 0;
      if ((rc = launch_cost(ca, d, mask_dtype, force_masks, st, 1u << first, false))) return rc;
      int32_t n[kClasses];
      if ((rc = wait_class_counts(cc_host, plan.nclass, first, st, n))) return rc;
      unsigned rest = 0;
      for (int c = 0; c < plan.nclass; ++c)
        if (c != first && n[c] != 0) rest |= 1u << c;
      // (the first class's own count: written with the others, read once;
      // not yet visible means no side stream)
      if (rest && !costs_only && first == kClasses - 1 && cc_host[first] > 0) {
        phase_first = first;
        rest_classes = rest;  // launched after the first class's finalize
      } else if (rest && (rc = launch_cost(ca, d, mask_dtype, force_masks, st, rest, false))) {
        return rc;
      }
    }
  }

  const bool use_softmax = p->use_softmax_label_loss != 0;
  AssignArgs aa;
  aa.cls_logits = cls_logits;
  aa.cls_dtype = cls_dtype;
  aa.cls_targets = cls_targets;
  aa.partials = ca.partials;
  aa.rowsum = ca.rowsum;
  aa.sched = ca.sched;
  aa.plan = plan;
  aa.ncols = pa.ncols;
  aa.slot_of_col = pa.slot_of_col;
  aa.colmap = pa.colmap;
  aa.sep = sep ? sep : (float*)(w + L.sep);
  if (cls_logits) {
    aa.out_bce = aa.sep;
    aa.out_dice = aa.sep + d.LB * d.Q * d.GT_out;
  } else {  // standalone pairwise BCE / dice: planes straight to the caller's outputs
    aa.out_bce = bce_out;
    aa.out_dice = dice_out;
  }
  aa.rowstat = (float*)(w + L.rowstat);
  aa.tot = costs_only ? nullptr : (float*)(w + L.tot);
  aa.tot64 = costs_only || lds_rows > 0 ? nullptr : (double*)(w + L.tot64);
  aa.tot_stride = ceil_div(d.Q * d.GT_out, 4) * 4;
  aa.rowIT = costs_only || !stats ? nullptr : (float*)(w + L.rowIT);
  aa.pred_to_gt = pred_to_gt;
  aa.pred_round = pred_round;
  aa.stats = stats;
  aa.img = (float*)(w + L.img);
  // the rest of the gradient's zero fill: extra workgroups of the assignment launch
  aa.fin_fill = fin_fill;
  aa.fill = (u32x4_t*)prefill + assign_from;
  aa.fill_n16 = fill_n16 - assign_from;
  aa.fill_tail = (unsigned char*)prefill + prefill_bytes / 16 * 16;
  aa.fill_ntail = (int64_t)(prefill_bytes % 16);
  aa.done = costs_only ? nullptr : (int*)(w + L.done);
  aa.fill_blocks = prefill_bytes
                       ? (int)std::min<int64_t>(kFillBlocks, std::max<int64_t>(1, ceil_div(aa.fill_n16, 256)))
                       : 0;
  aa.L = d.L; aa.B = d.B; aa.Q = d.Q; aa.C = d.C; aa.HW = d.HW; aa.Ht = d.Ht; aa.Wt = d.Wt;
  aa.GT_total = d.GT_total; aa.GT_out = d.GT_out; aa.bg = d.bg; aa.rtiles = d.rtiles;
  aa.rows = d.rows; aa.nslot = d.nslot; aa.N2 = (float)d.N2;
  aa.smooth = p->smooth; aa.sigmoid_scale = p->sigmoid_scale; aa.dice_scale = p->dice_scale;
  aa.cls_scale = p->cls_scale;
  aa.normalize = p->normalize_uncertainty != 0;
  aa.use_softmax = use_softmax;
  aa.force_cls = !costs_only && p->force_unmatched_class_to_background;
  aa.force_masks = force_masks;
  aa.void_idx = costs_only ? -1 : void_idx;
  aa.cls_gamma = p->cls_gamma;
  aa.cls_alpha = p->cls_alpha;
  // the label loss uses focal terms only in its sigmoid form
  aa.cls_ep = use_softmax ? make_elem_params(0.f, -1.f, 0.f, 0.f)
                          : make_elem_params(p->cls_gamma, p->cls_alpha, 0.f, 0.f);
  aa.mask_ep = mask_ep;
  aa.inf_thresh = p->inf_thresh;
  {
    const double x = p->inf_thresh;  // big_from, src/cpu/matching.cpp:71-83
    double big;
    if (!(x == x) || x == INFINITY || x == -INFINITY || x <= 0.0) big = 1e15;
    else {
      big = x * 0.5;
      if (big == INFINITY || big < 1e6) big = 1e15;
      if (big > 1e290) big = 1e290;
    }
    aa.big = big;
  }
  aa.topk = p->topk_matches;
  aa.strategy = (int)p->strategy_id;
  aa.costs_only = costs_only;
  aa.lds_rows = lds_rows;
  if (phase_first < 0 && d.LB > 0 && (rc = launch_finalize(aa, d, st))) return rc;
  if (costs_only) return ML_OK;
  // per-layer means and the matched-row list, after the assignment
  LayerArgs la;
  la.img = aa.img;
  la.layer = stats ? stats + d.LB * d.Q * ML_STATS : (float*)(w + L.layer);
  la.means = layer_means;
  la.pred_to_gt = pred_to_gt;
  la.list = saved ? (int*)(sv + SL.list) : nullptr;
  la.mrows = (int*)(w + L.mrows);
  la.L = d.L; la.B = d.B; la.Q = d.Q;
  la.num_masks = p->num_masks;
  la.force_masks = force_masks;
  la.force_cls = p->force_unmatched_class_to_background;
  la.has_void = void_idx >= 0;
  aa.layer_args = la;  // run by the last assignment workgroup
  if (phase_first >= 0) {
    // here: the first class's finalize, the other classes' contraction,
    // finalize (with its share of the gradient fill) and assignment (with
    // the assignment's share); side stream: the first class's assignment
    AssignArgs a1 = aa, a2 = aa;
    a1.reset_done = a2.reset_done = 0;  // zeroed by the column pass
    a1.phase_class = a2.phase_class = phase_first;
    a1.phase_in = 1;
    a2.phase_in = 0;
    a1.fin_fill = FillSlice();
    a1.fill_blocks = 0;
    a1.fill_n16 = a1.fill_ntail = 0;
    if ((rc = launch_finalize(a1, d, st, "finalize_early"))) return rc;
    if ((rc = side_acquire(side))) return rc;
    int rc1 = ML_OK, rc2 = ML_OK;
    if (hipEventRecord(side.fork, st) != hipSuccess || hipStreamWaitEvent(side.s, side.fork, 0) != hipSuccess)
      rc1 = fail(ML_ELAUNCH, "cannot fork the side stream");
    if (!rc1) rc1 = launch_assign(a1, d, side.s, "assign_early");
    {
      ProfScope ps_("cost_rest", st);
      rc2 = launch_cost(ca, d, mask_dtype, force_masks, st, rest_classes, false);
    }
    if (!rc2) rc2 = launch_finalize(a2, d, st);
    if (!rc2) rc2 = launch_assign(a2, d, st);
    // the join is enqueued whatever failed, so this stream's later work
    // (and the caller's frees) follow the side stream's
    const bool joined = hipEventRecord(side.join, side.s) == hipSuccess &&
                        hipStreamWaitEvent(st, side.join, 0) == hipSuccess;
    if (joined) side_release(side);
    if (rc1) return rc1;
    if (rc2) return rc2;
    if (!joined) {
      (void)hipStreamSynchronize(side.s);
      return fail(ML_ELAUNCH, "cannot join the side stream");
    }
  } else if (d.LB > 0) {
    if ((rc = launch_assign(aa, d, st))) return rc;
  } else {
    if (prefill_bytes) {
      ProfScope ps_("prefill", st);
      if ((rc = launch_zero_fill(prefill, prefill_bytes, st))) return rc;
    }
    if (d.L > 0 && (rc = launch_layer(la, st))) return rc;
  }
  return ML_OK;
}

// Workspace bytes of the matching forward with the packed cost plan fitted
// to `budget` (what forward_impl with packed = true and ws_bytes = budget
// needs) in `bytes`; the shape errors are
// those of ml_mask_matching_forward (ML_EINVAL for malformed shapes,
// ML_EUNSUPPORTED for shapes the assignment does not take).
int forward_packed_bytes(const ml_shape* s, const ml_params* p, int mask_dtype, size_t budget,
                         size_t& bytes) {
  Dims d;
  std::string err;
  bytes = 0;
  if (!make_dims(s, p->background_index, mask_dtype, d, err)) return fail(ML_EINVAL, err);
  if (!check_assign_dims(d, err)) return fail(ML_EUNSUPPORTED, err);
  const bool force_masks = p->force_unmatched_masks_to_empty != 0;
  const bool tab = mask_dtype == ML_BF16 && !d.counts_mode && g_use_lut && !force_masks;
  CostPlan plan = make_cost_plan(d, mask_dtype, tab);
  fit_cost_plan(plan, d, force_masks, budget);
  bytes = make_layout(d, force_masks, plan).total;
  return ML_OK;
}



}  // namespace ml

using namespace ml;

extern "C" {

const char* ml_last_error(void) { return g_err.c_str(); }

int ml_profile_enable(int enable) {
  std::lock_guard<std::mutex> g(g_prof_mu);
  if (enable && g_pool.size() < 512) {
    for (int i = 0; i < 512; ++i) {
      hipEvent_t e;
      if (hipEventCreate(&e) != hipSuccess) return fail(ML_ELAUNCH, "hipEventCreate failed");
      g_pool.push_back(e);
    }
  }
  g_prof_on = enable != 0;
  return ML_OK;
}

int ml_profile_reset(void) {
  std::lock_guard<std::mutex> g(g_prof_mu);
  for (auto& r : g_recs) {
    (void)hipEventSynchronize(r.b);
    g_pool.push_back(r.a);
    g_pool.push_back(r.b);
  }
  g_recs.clear();
  return ML_OK;
}

int ml_profile_read(const char* name, int64_t* launches, double* total_ms) {
  std::lock_guard<std::mutex> g(g_prof_mu);
  int64_t n = 0;
  double t = 0.0;
  for (auto& r : g_recs) {
    if (strcmp(r.name, name) != 0) continue;
    if (hipEventSynchronize(r.b) != hipSuccess) return fail(ML_ELAUNCH, "event sync failed");
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess) return fail(ML_ELAUNCH, "elapsed failed");
    ++n;
    t += ms;
  }
  *launches = n;
  *total_ms = t;
  return ML_OK;
}
int ml_version(void) { return 1; }

int ml_profile_stream_read(const void* p, size_t bytes, uint32_t* out, int grid, ml_stream_t stream) {
  if (!p || !out || bytes == 0 || bytes % 16 || ((uintptr_t)p & 15) || grid < 1 || grid > 65536)
    return fail(ML_EINVAL, "stream_read: bad arguments");
  return launch_stream_read(p, (int64_t)(bytes / 16), out, grid, (hipStream_t)stream);
}

int ml_any_equal(const int64_t* x, int64_t n, int64_t value, int32_t* flag, ml_stream_t stream) {
  if (n < 0 || (n > 0 && !x) || !flag) return fail(ML_EINVAL, "any_equal: bad arguments");
  return launch_any_equal(x, n, value, flag, (hipStream_t)stream);
}

size_t ml_saved_bytes(const ml_shape* s, const ml_params* p, int mask_dtype) {
  Dims d;
  std::string err;
  if (!make_dims(s, p->background_index, mask_dtype, d, err)) return fail(0, err);
  return saved_layout(d).total;
}

size_t ml_mask_matching_workspace_size(const ml_shape* s, const ml_params* p, int mask_dtype) {
  Dims d;
  std::string err;
  if (!make_dims(s, p->background_index, mask_dtype, d, err) || !check_assign_dims(d, err))
    return fail(0, err);
  return make_layout(d, p->force_unmatched_masks_to_empty != 0).total;
}

size_t ml_pairwise_mask_loss_workspace_size(const ml_shape* s, const ml_params* p,
                                            int mask_dtype) {
  Dims d;
  std::string err;
  if (!make_dims(s, p->background_index, mask_dtype, d, err)) return fail(0, err);
  return make_layout(d, false).total;
}

int ml_mask_matching_forward(const ml_shape* s, const ml_params* p, int mask_dtype,
                             const void* mask_logits, const int64_t* mask_targets, int cls_dtype,
                             const void* cls_logits, const int64_t* cls_targets,
                             int64_t* pred_to_gt, int64_t* pred_round, float* layer_means,
                             float* separate_costs, void* saved, void* grad_mask_prefill,
                             int32_t* void_found, ml_event_t void_ready, void* workspace,
                             size_t workspace_bytes, ml_stream_t stream) {
  int rc = check_params(p, s->C, true);
  if (rc) return rc;
  return forward_impl(s, p, mask_dtype, mask_logits, mask_targets, cls_dtype, cls_logits,
                      cls_targets, pred_to_gt, pred_round, layer_means, separate_costs, saved,
                      grad_mask_prefill, void_found, (hipEvent_t)void_ready, workspace,
                      workspace_bytes, (hipStream_t)stream, false, nullptr, nullptr, nullptr, 0,
                      0, false);
}

int ml_mask_matching_forward_polled(const ml_shape* s, const ml_params* p, int mask_dtype,
                                    const void* mask_logits, const int64_t* mask_targets,
                                    int cls_dtype, const void* cls_logits,
                                    const int64_t* cls_targets, int64_t* pred_to_gt,
                                    int64_t* pred_round, float* layer_means, float* separate_costs,
                                    void* saved, void* grad_mask_prefill, int32_t* void_found,
                                    ml_event_t void_ready, void* workspace, size_t workspace_bytes,
                                    ml_stream_t stream, int32_t* class_counts_dev,
                                    volatile int32_t* class_counts_host) {
  int rc = check_params(p, s->C, true);
  if (rc) return rc;
  if (!class_counts_dev || !class_counts_host)
    return fail(ML_EINVAL, "the class count words must not be null");
  return forward_impl(s, p, mask_dtype, mask_logits, mask_targets, cls_dtype, cls_logits,
                      cls_targets, pred_to_gt, pred_round, layer_means, separate_costs, saved,
                      grad_mask_prefill, void_found, (hipEvent_t)void_ready, workspace,
                      workspace_bytes, (hipStream_t)stream, false, nullptr, nullptr, nullptr, 0,
                      0, false, class_counts_dev, class_counts_host);
}

int ml_pairwise_mask_loss_forward(const ml_shape* s, const ml_params* p, int mask_dtype,
                                  const void* mask_logits, const int64_t* mask_targets,
                                  int cls_dtype, const void* cls_logits,
                                  const int64_t* cls_targets, float* separate_costs,
                                  void* workspace, size_t workspace_bytes, ml_stream_t stream) {
  int rc = check_params(p, s->C, false);
  if (rc) return rc;
  return forward_impl(s, p, mask_dtype, mask_logits, mask_targets, cls_dtype, cls_logits,
                      cls_targets, nullptr, nullptr, nullptr, separate_costs, nullptr, nullptr,
                      nullptr, nullptr, workspace, workspace_bytes, (hipStream_t)stream, true,
                      nullptr, nullptr, nullptr, 0, 0, false);
}

int ml_pairwise_sigmoid_dice_forward(const ml_shape* s, const ml_params* p, int dtype,
                                     const void* logits, const int64_t* targets, float* bce_out,
                                     float* dice_out, void* workspace, size_t workspace_bytes,
                                     ml_stream_t stream) {
  int rc = check_focal(p->mask_gamma, p->mask_alpha, "pairwise sigmoid");
  if (rc) return rc;
  if (!(p->uncertainty_gamma >= 0.f))
    return fail(ML_EINVAL, "uncertainty_gamma must be non-negative");
  if (!(p->uncertainty_gamma_min >= 0.f && p->uncertainty_gamma_min <= 1.f))
    return fail(ML_EINVAL, "uncertainty_gamma_min must be in [0, 1]");
  return forward_impl(s, p, dtype, logits, targets, ML_F32, nullptr, nullptr, nullptr, nullptr,
                      nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, workspace,
                      workspace_bytes, (hipStream_t)stream, true, bce_out, dice_out, nullptr, 0,
                      0, false);
}

// ---- point-sampling front end ------------------------------------------------
int ml_point_sample(int dtype, const void* input, const float* coords, int64_t N, int64_t C,
                    int64_t H, int64_t W, int64_t P, int64_t coords_batch, int align_corners,
                    void* out, ml_stream_t stream) {
  if (N < 0 || C < 0 || H <= 0 || W <= 0 || P < 0 || coords_batch <= 0)
    return fail(ML_EINVAL, "point_sample: invalid shape");
  if (!dtype_ok(dtype)) return fail(ML_EINVAL, "unsupported dtype");
  return launch_point_sample(dtype, input, coords, N, C, H, W, P, coords_batch, align_corners, out,
                             (hipStream_t)stream);
}

size_t ml_point_sample_backward_workspace_size(int dtype, int64_t N, int64_t C, int64_t H, int64_t W,
                                               int64_t P, int64_t coords_batch) {
  if (N < 0 || C < 0 || H <= 0 || W <= 0 || P < 0 || coords_batch <= 0 || !dtype_ok(dtype)) return 0;
  return point_sample_bwd_workspace(dtype, N, C, H, W, P, coords_batch);
}

int ml_point_sample_backward(int dtype, const void* grad_out, const float* coords, int64_t N,
                             int64_t C, int64_t H, int64_t W, int64_t P, int64_t coords_batch,
                             int align_corners, void* grad_input, float* workspace,
                             size_t workspace_bytes, ml_stream_t stream) {
  if (N < 0 || C < 0 || H <= 0 || W <= 0 || P < 0 || coords_batch <= 0)
    return fail(ML_EINVAL, "point_sample backward: invalid shape");
  if (!dtype_ok(dtype)) return fail(ML_EINVAL, "unsupported dtype");
  if (workspace_bytes < point_sample_bwd_workspace(dtype, N, C, H, W, P, coords_batch))
    return fail(ML_EWORKSPACE, "workspace too small");
  return launch_point_sample_backward(dtype, grad_out, coords, N, C, H, W, P, coords_batch,
                                      align_corners, grad_input, workspace, (hipStream_t)stream);
}

int ml_point_labels(const int64_t* targets, const float* coords, int64_t B, int64_t Ht, int64_t Wt,
                    int64_t P, int64_t* labels, ml_stream_t stream) {
  if (B < 0 || Ht <= 0 || Wt <= 0 || P < 0) return fail(ML_EINVAL, "point labels: invalid shape");
  return launch_point_labels(targets, coords, B, Ht, Wt, P, INT64_MAX, labels, nullptr, 0,
                             (hipStream_t)stream);
}

// The sampled-cost shape: s->H = 1, s->W = s->Wt = P (points), s->Ht = 1.
static bool points_shape_ok(const ml_shape* s, int64_t Hs, int64_t Ws) {
  return s->H == 1 && s->Ht == 1 && s->W == s->Wt && s->W > 0 && Hs > 0 && Ws > 0;
}

size_t ml_pairwise_points_workspace_size(const ml_shape* s, const ml_params* p, int dtype,
                                         int64_t Hs, int64_t Ws) {
  if (!points_shape_ok(s, Hs, Ws)) return 0;
  Dims d;
  std::string err;
  if (!make_dims(s, p->background_index, dtype, d, err)) return 0;
  return align256(make_layout(d, false).total) + (size_t)d.B * prep_blocks_map(Hs, Ws) * kPresWords * 4;
}

int ml_pairwise_sigmoid_dice_points_forward(const ml_shape* s, const ml_params* p, int dtype,
                                            const void* point_logits, const int64_t* targets,
                                            int64_t Hs, int64_t Ws, const float* coords,
                                            float* bce_out, float* dice_out, void* workspace,
                                            size_t workspace_bytes, ml_stream_t stream) {
  if (!points_shape_ok(s, Hs, Ws))
    return fail(ML_EINVAL, "sampled costs: the shape must be (L,B,C,1,P) with a (1,P) target row");
  if (!coords) return fail(ML_EINVAL, "sampled costs: point coordinates are required");
  int rc = check_focal(p->mask_gamma, p->mask_alpha, "pairwise sigmoid");
  if (rc) return rc;
  if (!(p->uncertainty_gamma >= 0.f))
    return fail(ML_EINVAL, "uncertainty_gamma must be non-negative");
  if (!(p->uncertainty_gamma_min >= 0.f && p->uncertainty_gamma_min <= 1.f))
    return fail(ML_EINVAL, "uncertainty_gamma_min must be in [0, 1]");
  return forward_impl(s, p, dtype, point_logits, targets, ML_F32, nullptr, nullptr, nullptr,
                      nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, workspace,
                      workspace_bytes, (hipStream_t)stream, true, bce_out, dice_out, coords, Hs,
                      Ws, false);
}

size_t ml_mask_matching_backward_workspace_size(const ml_shape* s, const ml_params* p,
                                                int mask_dtype) {
  Dims d;
  std::string err;
  if (!make_dims(s, p->background_index, mask_dtype, d, err)) return 0;
  size_t o = 0;
  o = align256(o + (d.counts_mode ? 0 : (size_t)d.B * d.HWp * 2));
  o = align256(o + (d.counts_mode ? (size_t)d.B * d.GT_total * d.HWp * d.cw : 0));
  o = align256(o + (size_t)d.B * 4);                // ncols
  o = align256(o + (size_t)d.B * d.nslot * 4);      // colmap
  o = align256(o + (size_t)d.B * d.GT_out * 4);     // slot_of_col
  o = align256(o + (size_t)d.L * ML_LAYERS * 4);    // layer
  return o;
}

int ml_mask_matching_backward(const ml_shape* s, const ml_params* p, const float* grad_mask,
                              const float* grad_dice, const float* grad_cls, int mask_dtype,
                              const void* mask_logits, const int64_t* mask_targets, int cls_dtype,
                              const void* cls_logits, const int64_t* cls_targets,
                              const int64_t* pred_to_gt, const void* saved,
                              int grad_prefilled, void* grad_mask_logits, void* grad_cls_logits,
                              void* workspace, size_t workspace_bytes, ml_stream_t stream) {
  int rc = check_params(p, s->C, true);
  if (rc) return rc;
  if (!dtype_ok(mask_dtype) || !dtype_ok(cls_dtype)) return fail(ML_EINVAL, "unsupported dtype");
  Dims d;
  std::string err;
  if (!make_dims(s, p->background_index, mask_dtype, d, err)) return fail(ML_EINVAL, err);
  if (workspace_bytes < ml_mask_matching_backward_workspace_size(s, p, mask_dtype))
    return fail(ML_EWORKSPACE, "workspace too small");
  if (grad_prefilled && (!saved || p->force_unmatched_masks_to_empty))
    return fail(ML_EINVAL, "a prefilled gradient needs the saved state and unforced unmatched masks");
  const SavedLayout SL = saved_layout(d);
  const unsigned char* sv = (const unsigned char*)saved;
  const float* stats = saved ? (const float*)(sv + SL.stats) : nullptr;
  hipStream_t st = (hipStream_t)stream;
  unsigned char* w = (unsigned char*)workspace;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t r = o;
    o = align256(o + bytes);
    return r;
  };
  PrepArgs pa;
  pa.lab16 = (uint16_t*)(w + take(d.counts_mode ? 0 : (size_t)d.B * d.HWp * 2));
  pa.counts = (uint8_t*)(w + take(d.counts_mode ? (size_t)d.B * d.GT_total * d.HWp * d.cw : 0));
  pa.cw = d.cw;
  pa.pbits = nullptr;  // labels only
  pa.ncols = (int*)(w + take((size_t)d.B * 4));
  pa.colmap = (int*)(w + take((size_t)d.B * d.nslot * 4));
  pa.slot_of_col = (int*)(w + take((size_t)d.B * d.GT_out * 4));
  float* layer_ws = (float*)(w + take((size_t)d.L * ML_LAYERS * 4));
  pa.targets = mask_targets;
  pa.B = d.B; pa.H = d.H; pa.W = d.W; pa.Ht = d.Ht; pa.Wt = d.Wt; pa.s = d.s; pa.HWp = d.HWp;
  pa.GT_total = d.GT_total; pa.GT_out = d.GT_out; pa.bg = d.bg; pa.nslot = d.nslot;
  pa.sched = nullptr;
  pa.L = d.L; pa.rtiles = d.rtiles; pa.plan = CostPlan{};
  // the forward's saved state holds the compact label map for s == 1
  const bool saved_labels = saved && !d.counts_mode;
  if (saved_labels) pa.lab16 = (uint16_t*)(sv + SL.lab16);
  else if (d.B > 0 && (rc = launch_prep(pa, d, st))) return rc;

  const int64_t void_idx =
      (p->void_class_index >= 0 && p->void_class_index < d.C) ? p->void_class_index : -1;
  const float* layer;
  if (stats) {
    layer = stats + d.LB * d.Q * ML_STATS;
  } else {
    if (d.L > 0 &&
        (rc = launch_layer_from_p2g(pred_to_gt, layer_ws, d.L, d.B, d.Q, p->num_masks,
                                    p->force_unmatched_masks_to_empty,
                                    p->force_unmatched_class_to_background, void_idx >= 0, st)))
      return rc;
    layer = layer_ws;
  }
  BwdArgs ba;
  ba.logits = mask_logits;
  ba.dtype = mask_dtype;
  ba.lab16 = d.counts_mode ? nullptr : pa.lab16;
  ba.counts = d.counts_mode ? pa.counts : nullptr;
  ba.cw = d.cw;
  ba.pred_to_gt = pred_to_gt;
  ba.stats = stats;
  ba.list = grad_prefilled ? (const int*)(sv + SL.list) : nullptr;
  ba.layer = layer;
  ba.g_mask = grad_mask;
  ba.g_dice = grad_dice;
  ba.g_cls = grad_cls;
  ba.grad = grad_mask_logits;
  ba.cls_logits = cls_logits;
  ba.cls_dtype = cls_dtype;
  ba.cls_targets = cls_targets;
  ba.grad_cls = grad_cls_logits;
  ba.L = d.L; ba.B = d.B; ba.Q = d.Q; ba.HW = d.HW; ba.HWp = d.HWp; ba.C = d.C;
  ba.GT_total = d.GT_total; ba.bg = d.bg; ba.Ht = d.Ht; ba.Wt = d.Wt; ba.N2 = (float)d.N2;
  ba.smooth = p->smooth; ba.sigmoid_scale = p->sigmoid_scale; ba.dice_scale = p->dice_scale;
  ba.cls_scale = p->cls_scale; ba.normalize = p->normalize_uncertainty != 0;
  ba.force_masks = p->force_unmatched_masks_to_empty != 0;
  ba.force_cls = p->force_unmatched_class_to_background != 0;
  ba.use_softmax = p->use_softmax_label_loss != 0;
  ba.void_idx = void_idx;
  ba.mask_ep = make_elem_params(p->mask_gamma, p->mask_alpha, p->uncertainty_gamma,
                                p->uncertainty_gamma_min);
  ba.cls_ep = ba.use_softmax ? make_elem_params(0.f, -1.f, 0.f, 0.f)
                             : make_elem_params(p->cls_gamma, p->cls_alpha, 0.f, 0.f);
  ba.cls_gamma = ba.use_softmax ? 0.f : p->cls_gamma;
  ba.cls_fused = 0;
  return launch_bwd(ba, d, st);
}

// ---- dense (non-pairwise) sigmoid CE / dice -------------------------------------
namespace {
struct DensePlan {
  Dims d;             // B, H, W, Ht, Wt, s, HW, HWp, counts_mode; GT_total := C
  size_t tgt_bytes, partial_off, total;
};

bool dense_plan(const ml_dense_shape* s, bool dice, bool backward, DensePlan& P,
                std::string& err) {
  if (!s || s->L < 0 || s->B < 0 || s->C < 0 || s->H <= 0 || s->W <= 0) {
    err = "dense loss: invalid shape";
    return false;
  }
  Dims& d = P.d;
  d = Dims{};
  d.L = s->L; d.B = s->B; d.Q = 0; d.H = s->H; d.W = s->W; d.Ht = s->Ht; d.Wt = s->Wt;
  d.C = s->C; d.GT_total = s->C;
  if (d.Ht % d.H != 0 || d.Wt % d.W != 0 || d.Ht / d.H != d.Wt / d.W || d.Ht == 0) {
    err = "High-res dims must be the same integer multiple of the low-res dims";
    return false;
  }
  d.s = d.Ht / d.H;
  if (d.s > 255) {
    err = "target/logit scale factors above 255 are not supported (per-cell counts are 16-bit)";
    return false;
  }
  if (d.C > 65535) {
    err = "at most 65535 classes are supported";
    return false;
  }
  d.N2 = d.s * d.s;
  d.LB = d.L * d.B;
  d.HW = d.H * d.W;
  d.HWp = ceil_div(d.HW, kStep) * kStep;
  d.counts_mode = d.s > 1;
  d.cw = d.s >= 16 ? 2 : 1;
  P.tgt_bytes = align256(d.counts_mode ? (size_t)d.B * d.C * d.HWp * d.cw : (size_t)d.B * d.HWp * 2);
  P.partial_off = P.tgt_bytes;
  P.total = P.tgt_bytes + (backward ? 0 : align256(dense_partials_bytes(d.L, d.B, d.C, d.HW, dice)));
  return true;
}

int dense_prep(const DensePlan& P, const int64_t* targets, unsigned char* w, DenseArgs& a,
               hipStream_t st) {
  const Dims& d = P.d;
  PrepArgs pa{};
  pa.targets = targets;
  pa.lab16 = d.counts_mode ? nullptr : (uint16_t*)w;
  pa.counts = d.counts_mode ? (uint8_t*)w : nullptr;
  pa.cw = d.cw;
  pa.pbits = nullptr;
  pa.B = d.B; pa.H = d.H; pa.W = d.W; pa.Ht = d.Ht; pa.Wt = d.Wt; pa.s = d.s; pa.HWp = d.HWp;
  pa.GT_total = d.C; pa.GT_out = d.C; pa.bg = d.C;
  a.lab16 = pa.lab16;
  a.counts = pa.counts;
  a.cw = d.cw;
  a.L = d.L; a.B = d.B; a.C = d.C; a.HW = d.HW; a.HWp = d.HWp; a.HtWt = d.Ht * d.Wt;
  a.N2 = (float)d.N2;
  if (d.B == 0) return ML_OK;
  return launch_prep(pa, d, st);
}
}  // namespace

size_t ml_dense_loss_workspace_size(const ml_dense_shape* s, int dtype, int dice, int backward) {
  DensePlan P;
  std::string err;
  if (!dtype_ok(dtype) || !dense_plan(s, dice != 0, backward != 0, P, err)) return 0;
  return P.total;
}

static int dense_call(const ml_dense_shape* s, int dtype, bool dice, bool backward,
                      const int64_t* targets, void* ws, size_t ws_bytes, DenseArgs& a,
                      hipStream_t st) {
  if (!dtype_ok(dtype)) return fail(ML_EINVAL, "unsupported dtype");
  DensePlan P;
  std::string err;
  if (!dense_plan(s, dice, backward, P, err)) return fail(ML_EINVAL, err);
  if (ws_bytes < P.total) return fail(ML_EWORKSPACE, "workspace too small");
  unsigned char* w = (unsigned char*)ws;
  a.dtype = dtype;
  a.partials = backward ? nullptr : (double*)(w + P.partial_off);
  int rc = dense_prep(P, targets, w, a, st);
  if (rc) return rc;
  return launch_dense(a, dice, backward, st);
}

int ml_sigmoid_ce_forward(const ml_dense_shape* s, int dtype, const void* logits,
                          const int64_t* targets, float num_masks, float scale, float gamma,
                          float alpha, float* loss, void* workspace, size_t workspace_bytes,
                          ml_stream_t stream) {
  int rc = check_focal(gamma, alpha, "sigmoid_ce");
  if (rc) return rc;
  DenseArgs a{};
  a.logits = logits;
  a.ep = make_elem_params(gamma, alpha, 0.f, 0.f);
  a.scale = scale;
  a.num_masks = (double)num_masks;
  a.loss = loss;
  return dense_call(s, dtype, false, false, targets, workspace, workspace_bytes, a,
                    (hipStream_t)stream);
}

int ml_sigmoid_ce_backward(const ml_dense_shape* s, int dtype, const float* grad_out,
                           const void* logits, const int64_t* targets, float num_masks,
                           float scale, float gamma, float alpha, void* grad, void* workspace,
                           size_t workspace_bytes, ml_stream_t stream) {
  int rc = check_focal(gamma, alpha, "sigmoid_ce");
  if (rc) return rc;
  DenseArgs a{};
  a.logits = logits;
  a.ep = make_elem_params(gamma, alpha, 0.f, 0.f);
  a.scale = scale;
  a.num_masks = (double)num_masks;
  a.grad_out = grad_out;
  a.grad = grad;
  return dense_call(s, dtype, false, true, targets, workspace, workspace_bytes, a,
                    (hipStream_t)stream);
}

int ml_dice_loss_forward(const ml_dense_shape* s, int dtype, const void* logits,
                         const int64_t* targets, float smooth, float num_masks, float scale,
                         float* loss, float* I, float* P, float* T, void* workspace,
                         size_t workspace_bytes, ml_stream_t stream) {
  DenseArgs a{};
  a.logits = logits;
  a.smooth = smooth;
  a.scale = scale;
  a.num_masks = (double)num_masks;
  a.loss = loss;
  a.I_out = I;
  a.P_out = P;
  a.T_out = T;
  return dense_call(s, dtype, true, false, targets, workspace, workspace_bytes, a,
                    (hipStream_t)stream);
}

int ml_dice_loss_backward(const ml_dense_shape* s, int dtype, const float* grad_out,
                          const void* logits, const int64_t* targets, const float* I,
                          const float* P, const float* T, float smooth, float num_masks,
                          float scale, void* grad, void* workspace, size_t workspace_bytes,
                          ml_stream_t stream) {
  DenseArgs a{};
  a.logits = logits;
  a.smooth = smooth;
  a.scale = scale;
  a.num_masks = (double)num_masks;
  a.grad_out = grad_out;
  a.I_in = I;
  a.P_in = P;
  a.T_in = T;
  a.grad = grad;
  return dense_call(s, dtype, true, true, targets, workspace, workspace_bytes, a,
                    (hipStream_t)stream);
}

int ml_pairwise_label_loss_forward(int64_t L, int64_t B, int64_t Q, int64_t C, int64_t GT_total,
                                   int cls_dtype, const void* cls_logits,
                                   const int64_t* cls_targets, int64_t background_index,
                                   float scale, float gamma, float alpha, int use_softmax,
                                   float* out, ml_stream_t stream) {
  if (!dtype_ok(cls_dtype)) return fail(ML_EINVAL, "unsupported dtype");
  if (!use_softmax) {
    int rc = check_focal(gamma, alpha, "label");
    if (rc) return rc;
  }
  const bool skip = background_index >= 0 && background_index < GT_total;
  const int64_t bg = background_index >= 0 ? background_index : GT_total;
  const int64_t GT_out = GT_total - (skip ? 1 : 0);
  const ElemParams ep = use_softmax ? make_elem_params(0.f, -1.f, 0.f, 0.f)
                                    : make_elem_params(gamma, alpha, 0.f, 0.f);
  return launch_label_cost(cls_logits, cls_dtype, cls_targets, L, B, Q, C, GT_total, GT_out, bg,
                           scale, ep, use_softmax, out, (hipStream_t)stream);
}

}  // extern "C"
