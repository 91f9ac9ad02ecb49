// Per-image finalize + assignment + matched-loss forward partials.
//
// One workgroup (4 waves) per (layer, image):
//   1. per-query statistics: uncertainty normaliser S and mass P (from the
//      ones column of the cost contraction), label-loss row terms, unmatched
//      penalties (src/cuda/mask_matching_forward.cu:125-277);
//   2. every (query, column) cost: bce, dice (src/cuda/pw_mask.cu:299-305),
//      label cost (src/cuda/pw_sigmoid_label_loss.cu:76-105,
//      src/cuda/pw_softmax_label_loss.cu:84-102), total = (bce+dice)+cls as
//      float (src/cpu/matching.cpp:665), column validity
//      (src/cpu/matching.cpp:497-511);
//   3. assignment on wave 0 in float64 (src/cpu/matching.cpp:95-463): the
//      e-maxx shortest augmenting path with the reference's operation order
//      cur = (c - u[i0]) - v[j], strict '<' updates and lowest-index argmin,
//      so it returns the reference's assignment bit for bit on the same cost
//      matrix;
//   4. pred_round ranking by (cost, query) (src/cpu/matching.cpp:533-565),
//      per-image matched-loss sums (src/cuda/mask_matching_forward.cu:63-71)
//      and per-query statistics for the fused backward.
#include <atomic>
#include <mutex>
#include <type_traits>

#include "ml_internal.h"

namespace ml {

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ double wave_min_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmin(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float cls_elem(const void* p, int dt, int64_t i) {
  if (dt == ML_F32) return ((const float*)p)[i];
  const uint16_t h = ((const uint16_t*)p)[i];
  if (dt == ML_BF16) return __uint_as_float(((uint32_t)h) << 16);
  return (float)__builtin_bit_cast(_Float16, h);
}

template <int DT>
__device__ __forceinline__ float cls_at(const void* p, int64_t i) {
  if constexpr (DT == ML_F32) return ((const float*)p)[i];
  const uint16_t h = ((const uint16_t*)p)[i];
  if constexpr (DT == ML_BF16) return __uint_as_float(((uint32_t)h) << 16);
  return (float)__builtin_bit_cast(_Float16, h);
}

// Reference float32 formulas for one label logit (mask_matching_forward.cu:195-218).
struct ClsTerm {
  float neg, pos;
};
__device__ __forceinline__ ClsTerm cls_terms(float z, const ElemParams& ep) {
  const Sig s = sig_terms(z);
  float mn, mp;
  focal_mods(s, ep, mn, mp);
  ClsTerm t;
  t.neg = ep.an * mn * s.cn;
  t.pos = ep.ap * mp * s.cp;
  return t;
}

struct SmemLayout {
  size_t contrib, colok, vcols, preds, p, way, u, hrows, asg, costL, total;
};

__host__ __device__ inline SmemLayout smem_layout(int64_t Q, int64_t GTo, int64_t lds_rows) {
  SmemLayout s;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    size_t r = o;
    o += (bytes + 15) & ~size_t(15);
    return r;
  };
  s.contrib = take(Q * 4 * 4);
  s.colok = take((GTo + 1) * 4);
  s.vcols = take((GTo + 1) * 4);
  s.preds = take((Q + 1) * 4);
  s.p = take((Q + 1) * 4);
  s.way = take((Q + 1) * 4);
  s.u = take((Q + 1) * 8);
  s.hrows = take((Q + 1) * 4);
  s.asg = take((Q + 1) * 4);
  s.costL = o;
  if (lds_rows > 0) take(lds_rows * Q * 4);
  s.total = o;
  return s;
}

__device__ __forceinline__ bool cost_ok(double c, double thr) { return isfinite(c) && c < thr; }

// ---------------------------------------------------------------------------
// Finalize: one wave per (l, b, q) row.  Sums the K-split partials of every
// used column slot, forms bce and dice (src/cuda/pw_mask.cu:299-305), the
// label cost (src/cuda/pw_sigmoid_label_loss.cu:76-105,
// src/cuda/pw_softmax_label_loss.cu:84-102), +inf for empty GTs or invalid
// classes, and the row terms used later: normaliser S, mass P, and the
// unmatched-query penalties (src/cuda/mask_matching_forward.cu:125-277).
// ---------------------------------------------------------------------------
// Each row is a short chain of dependent memory round trips, and the grid
// runs in a single round, so the kernel takes as long as one chain: every
// load that does not depend on an earlier one is issued up front (column
// count, schedule entries of every class, class logits, the output columns'
// slots and targets), then the K-split partials together with the class
// logits of the targets, then the stores.
// Register forms of finalize: (class logits, output columns) held per lane
constexpr int kFinCls = 3;       // C <= 192
constexpr int kFinCols = 2;      // GT_out <= 128
constexpr int kFinColsWide = 4;  // GT_out <= 256, class logits streamed (NC = 0)
constexpr int kFinClsBatch = 8;  // streamed class logits loaded per lane and batch
constexpr int kFinClsWide = 20;  // C <= 1280 in registers with up to 64 kFinColsWide output columns
constexpr int kFinSplits = 12;  // K-splits loaded per lane and batch
constexpr int kFinSplits4 = 9;  // the same for four-plane partials (same registers)

// Sum the K-split partials k0, k0 + step, ... of slot s in split order.  The
// loads of a batch are unconditional (indices clamped to the last split) so
// all of them are in flight together.
__device__ __forceinline__ void sum_splits(const RowPartials& rp, int s, int k0, int step,
                                           float& v0, float& v1, float& v2) {
  float a0 = 0.f, a1 = 0.f, a2 = 0.f;
  for (int base = k0; base < rp.KS; base += kFinSplits * step) {
    float x0[kFinSplits], x1[kFinSplits], x2[kFinSplits];
#pragma unroll
    for (int u = 0; u < kFinSplits; ++u) {
      const int ks = min(base + u * step, rp.KS - 1);
      const float* P = rp.p0 + (int64_t)ks * rp.ks_stride + s;
      x0[u] = P[0];
      x1[u] = P[rp.plane];
      x2[u] = P[2 * rp.plane];
    }
#pragma unroll
    for (int u = 0; u < kFinSplits; ++u) {
      if (base + u * step < rp.KS) {
        a0 += x0[u];
        a1 += x1[u];
        a2 += x2[u];
      }
    }
  }
  v0 = a0;
  v1 = a1;
  v2 = a2;
}

// The same for four-plane partials (slot sums of A_neg, A_pos, A_p, A_w).
__device__ __forceinline__ void sum_splits4(const RowPartials& rp, int s, float& v0, float& v1,
                                            float& v2, float& v3) {
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  for (int base = 0; base < rp.KS; base += kFinSplits4) {
    float x0[kFinSplits4], x1[kFinSplits4], x2[kFinSplits4], x3[kFinSplits4];
#pragma unroll
    for (int u = 0; u < kFinSplits4; ++u) {
      const int ks = min(base + u, rp.KS - 1);
      const float* P = rp.p0 + (int64_t)ks * rp.ks_stride + s;
      x0[u] = P[0];
      x1[u] = P[rp.plane];
      x2[u] = P[2 * rp.plane];
      x3[u] = P[3 * rp.plane];
    }
#pragma unroll
    for (int u = 0; u < kFinSplits4; ++u) {
      if (base + u < rp.KS) {
        a0 += x0[u];
        a1 += x1[u];
        a2 += x2[u];
        a3 += x3[u];
      }
    }
  }
  v0 = a0;
  v1 = a1;
  v2 = a2;
  v3 = a3;
}

// Exclusive prefix (UP) or suffix sum of v over the wave's lanes, in a fixed
// order.
template <bool UP>
__device__ __forceinline__ float wave_excl_scan(float v, int lane) {
  float x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const float y = UP ? __shfl_up(x, d, 64) : __shfl_down(x, d, 64);
    if (UP ? lane >= d : lane + d < 64) x += y;
  }
  const float e = UP ? __shfl_up(x, 1, 64) : __shfl_down(x, 1, 64);
  return (UP ? lane >= 1 : lane + 1 < 64) ? e : 0.f;
}

// Latency-bound: at least four waves per SIMD (at most 128 registers).
// CDT: dtype of the class logits.  FAST (chosen on the host): class logits
// present and 1 <= GT_out <= 64 NG, so the output columns' slots and targets
// fit in registers and every load of the first two round trips is
// unconditional (indices clamped into range); with NC > 0 (C <= 64 NC) the
// row's class logits are held in registers too, else they are streamed in
// batches of kFinClsBatch loads per lane.
template <int CDT, bool FAST, int NC = kFinCls, int NG = kFinCols>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NC > 8 ? 3 : 4))) void finalize_kernel(AssignArgs a) {
  if (blockIdx.x == 0 && threadIdx.x == 0) {  // the assignment's finish count
    if (a.done && a.reset_done) *a.done = 0;
  }
  __shared__ float sl[4][4][256 + 16];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // 32-bit index arithmetic: the host checks L * B * Q < 2^31
  const uint32_t nrows = (uint32_t)(a.L * a.B * a.Q), nrow_blocks = (nrows + 3u) / 4u;
  if (blockIdx.x >= nrow_blocks) {  // the launch's slice of the gradient's zero fill
    fill_slice(a.fin_fill, blockIdx.x - nrow_blocks);
    return;
  }
  const uint32_t row32 = blockIdx.x * 4u + (uint32_t)wave;
  if (row32 >= nrows) return;
  const uint32_t lb32 = row32 / (uint32_t)a.Q;
  const int64_t row = row32, lb = lb32, q = row32 - lb32 * (uint32_t)a.Q, b = lb32 % (uint32_t)a.B;
  const int64_t GTo = a.GT_out, C = a.C;
  const bool labels = FAST || a.cls_logits != nullptr;
  constexpr bool kClsRegs = FAST && NC > 0;
  const int64_t zb = row * C;
  const int64_t void_idx = a.void_idx;
  const bool has_void = void_idx >= 0;
  const bool softmax_bg = a.use_softmax && a.force_cls && has_void;

  // round trip 1: nothing here depends on another load
  const int G = a.ncols[b];
  const uint32_t rtile = (uint32_t)q / (uint32_t)a.rows;
  const int qin = (int)((uint32_t)q - rtile * (uint32_t)a.rows);
  const int64_t task = lb * a.rtiles + rtile;
  const int64_t tidx = a.sched[kSchedList + kClasses * a.plan.ntasks + task];
  int ksc[kClasses], nc[kClasses];
#pragma unroll
  for (int c = 0; c < kClasses; ++c) {
    ksc[c] = a.sched[kClasses + c];
    nc[c] = a.sched[c];
  }
  float zc[NC > 0 ? NC : 1] = {};
  int oslot[NG] = {};
  int64_t oy[NG] = {};
  float zy[NG] = {};
  float zv = 0.f;
  if constexpr (FAST) {
    if constexpr (kClsRegs) {
#pragma unroll
      for (int j = 0; j < NC; ++j) zc[j] = cls_at<CDT>(a.cls_logits, zb + min((int64_t)lane + 64 * j, C - 1));
    }
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const int64_t cc = min((int64_t)lane + 64 * j, GTo - 1);
      oslot[j] = a.slot_of_col[b * GTo + cc];
      oy[j] = a.cls_targets[b * a.GT_total + cc + (cc >= a.bg ? 1 : 0)];
    }
    zv = cls_at<CDT>(a.cls_logits, zb + (has_void ? void_idx : 0));
  } else if (labels && a.use_softmax && has_void) {
    zv = cls_at<CDT>(a.cls_logits, zb + void_idx);
  }
  // (softmax with forced background always has a void index: the host checks it)
  const bool need_zv = labels && a.use_softmax && has_void;

  // round trip 2: the partials (need the column class) and the targets' logits
  if (!in_phase(a.phase_class, a.phase_in, G)) return;  // another launch's image
  const int ci = class_of(G + 1);
  int KS = ksc[0], n_ci = nc[0];
#pragma unroll
  for (int c = 1; c < kClasses; ++c)
    if (ci == c) {
      KS = ksc[c];
      n_ci = nc[c];
    }
  const RowPartials rp = row_partials_at(a.partials, a.plan, ci, tidx, KS, n_ci, qin, a.rows);
  if constexpr (FAST) {
#pragma unroll
    for (int j = 0; j < NG; ++j) zy[j] = cls_at<CDT>(a.cls_logits, zb + min(max(oy[j], (int64_t)0), C - 1));
  }
  const int nsl = G + 1;  // GT columns + the ones column
  if (nsl <= 32) {
    // two lanes per slot, each summing every other K-split; fixed-order combine
    const int s = lane & 31, half = lane >> 5;
    float v0 = 0.f, v1 = 0.f, v2 = 0.f;
    if (s < nsl) sum_splits(rp, s, half, 2, v0, v1, v2);
    v0 += __shfl_xor(v0, 32, 64);
    v1 += __shfl_xor(v1, 32, 64);
    v2 += __shfl_xor(v2, 32, 64);
    if (half == 0 && s < nsl) {
      sl[wave][0][s] = v0;
      sl[wave][1][s] = v1;
      sl[wave][2][s] = v2;
    }
  } else if (a.plan.planes[ci] == 3) {
    for (int s = lane; s < nsl; s += 64) {
      float v0 = 0.f, v1 = 0.f, v2 = 0.f;
      sum_splits(rp, s, 0, 1, v0, v1, v2);
      sl[wave][0][s] = v0;
      sl[wave][1][s] = v1;
      sl[wave][2][s] = v2;
    }
  } else {
    // slot sums N, Pos, I, T of slots 0..G (slot G: cells of no column)
    for (int s = lane; s < nsl; s += 64) {
      float v0 = 0.f, v1 = 0.f, v2 = 0.f, v3 = 0.f;
      sum_splits4(rp, s, v0, v1, v2, v3);
      sl[wave][0][s] = v0;
      sl[wave][3][s] = v1;
      sl[wave][1][s] = v2;
      sl[wave][2][s] = v3;
    }
    wave_sync();
    // bce numerator of slot g: the A_neg sums of every other slot (cells
    // outside g) plus g's A_pos sum, from an exclusive prefix and suffix of
    // the N sums (non-negative terms, no cancellation); P and S: the I and T
    // sums over all slots.  Lane l takes slots 4l .. 4l + 3.
    float nv[4], iv = 0.f, tv = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int s = 4 * lane + k;
      const bool ok = s < nsl;
      nv[k] = ok ? sl[wave][0][s] : 0.f;
      iv += ok ? sl[wave][1][s] : 0.f;
      tv += ok ? sl[wave][2][s] : 0.f;
    }
    float in[4], sf[4];  // within the lane: inclusive prefix and suffix
    in[0] = nv[0];
#pragma unroll
    for (int k = 1; k < 4; ++k) in[k] = in[k - 1] + nv[k];
    sf[3] = nv[3];
#pragma unroll
    for (int k = 2; k >= 0; --k) sf[k] = nv[k] + sf[k + 1];
    const float pre = wave_excl_scan<true>(in[3], lane), suf = wave_excl_scan<false>(sf[0], lane);
    const float Ptot = wave_sum(iv), Stot = wave_sum(tv);
    wave_sync();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int s = 4 * lane + k;
      if (s < G) {
        const float before = k > 0 ? pre + in[k - 1] : pre;
        const float after = k < 3 ? suf + sf[k + 1] : suf;
        sl[wave][0][s] = (before + after) + sl[wave][3][s];
      }
    }
    if (lane == 0) {
      sl[wave][1][G] = Ptot;
      sl[wave][2][G] = Stot;
    }
  }

  // label row term and unmatched class penalty (none without class logits:
  // the standalone pairwise BCE / dice operators)
  // f(c, z) over this lane's classes c = lane, lane + 64, ... in that order
  auto for_cls = [&](auto&& f) {
    if constexpr (kClsRegs) {
#pragma unroll
      for (int j = 0; j < NC; ++j)
        if (lane + 64 * j < C) f((int64_t)lane + 64 * j, zc[j]);
    } else {
      for (int64_t c0 = lane; c0 < C; c0 += 64 * kFinClsBatch) {
        float z[kFinClsBatch];  // the batch's loads in flight together
#pragma unroll
        for (int u = 0; u < kFinClsBatch; ++u) z[u] = cls_at<CDT>(a.cls_logits, zb + min(c0 + 64 * u, C - 1));
#pragma unroll
        for (int u = 0; u < kFinClsBatch; ++u)
          if (c0 + 64 * u < C) f(c0 + 64 * u, z[u]);
      }
    }
  };
  float rowv = 0.f, pen = 0.f;
  if (!labels) {
  } else if (a.use_softmax) {
    float m = -INFINITY;
    for_cls([&](int64_t, float z) { m = fmaxf(m, z); });
    m = wave_max(m);
    float se = 0.f;
    for_cls([&](int64_t, float z) { se += __expf(z - m); });
    se = wave_sum(se);
    rowv = __logf(fmaxf(se, 1e-20f)) + m;
    if (need_zv) {
      // softmax CE towards void when forcing background; otherwise the
      // sigmoid BCE of the void channel (mask_matching_forward.cu:146-218)
      pen = softmax_bg ? (rowv - zv) * a.cls_scale : sig_terms(zv).cp * a.cls_scale;
    }
  } else {
    float base = 0.f, vpos = 0.f, vneg = 0.f;
    for_cls([&](int64_t c, float z) {
      const ClsTerm t = cls_terms(z, a.cls_ep);
      base += t.neg;
      if (c == void_idx) {
        vpos = t.pos;
        vneg = t.neg;
      }
    });
    base = wave_sum(base);
    vpos = wave_sum(vpos);
    vneg = wave_sum(vneg);
    rowv = base;
    if (a.force_cls) {
      const float invC = C > 0 ? 1.f / (float)C : 0.f;
      pen = base * invC;
      if (has_void && C > 0) pen += (vpos - vneg) * invC;
    } else if (has_void) {
      pen = vpos;
    }
    pen *= a.cls_scale;
  }
  wave_sync();
  if (a.rowIT) {  // summed intersection / target mass of every real slot (backward statistics)
    float2* it = (float2*)a.rowIT + row * a.nslot;
    for (int s = lane; s < G; s += 64) it[s] = make_float2(sl[wave][1][s], sl[wave][2][s]);
  }
  float S = sl[wave][2][G];
  const float P = sl[wave][1][G];
  if (!a.normalize) S = (float)(a.Ht * a.Wt);
  S = fmaxf(S, kEps);

  // all output columns of this row
  const int64_t term = a.L * a.B * a.Q * GTo;
  auto emit = [&](int64_t c, int slot, int64_t y, float zyc) {
    float bce = INFINITY, dice = INFINITY, cls;
    if (slot >= 0) {
      bce = sl[wave][0][slot] / S * a.sigmoid_scale;
      dice = (1.f - (2.f * sl[wave][1][slot] + a.smooth) / (P + sl[wave][2][slot] + a.smooth)) *
             a.dice_scale;
    }
    if (!labels) {
      cls = 0.f;
    } else if (y < 0 || y >= C) {
      cls = INFINITY;
    } else if (a.use_softmax) {
      cls = (rowv - zyc) * a.cls_scale;
    } else {
      const ClsTerm t = cls_terms(zyc, a.cls_ep);
      cls = (rowv + (t.pos - t.neg)) * (1.f / (float)C) * a.cls_scale;
    }
    const int64_t o = row * GTo + c;
    if (a.out_bce) a.out_bce[o] = bce;
    if (a.out_dice) a.out_dice[o] = dice;
    if (labels) a.sep[2 * term + o] = cls;
    // total cost, matching.cpp:665, stored [column][query]: the assignment
    // reads cost rows of one GT across all queries.  A NaN stands for every
    // non-finite total, so the assignment tests a cost with one comparison
    // (raw < inf_thresh is cost_ok(raw)).
    if (a.tot) {
      const float t = (bce + dice) + cls;
      a.tot[lb * a.tot_stride + c * a.Q + q] = __builtin_isfinite(t) ? t : __builtin_nanf("");
    }
  };
  if constexpr (FAST) {
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const int64_t c = lane + 64 * j;
      if (c < GTo) emit(c, oslot[j], oy[j], zy[j]);
    }
  } else {
    for (int64_t c = lane; c < GTo; c += 64) {
      const int slot = a.slot_of_col[b * GTo + c];
      const int64_t y = labels ? a.cls_targets[b * a.GT_total + c + (c >= a.bg ? 1 : 0)] : 0;
      const float zyc = (labels && y >= 0 && y < C) ? cls_at<CDT>(a.cls_logits, zb + y) : 0.f;
      emit(c, slot, y, zyc);
    }
  }
  if (lane == 0 && a.rowstat) {
    float mp = 0.f, dp = 0.f;
    if (a.force_masks) {
      float ub = 0.f, up = 0.f;
      for (int ks = 0; ks < rp.KS; ++ks) {
        const float* rs = a.rowsum + ((rp.slot0 + ks * rp.slot_stride) * a.rows + q % a.rows) * 2;
        ub += rs[0];
        up += rs[1];
      }
      const float psum = up * a.N2;
      mp = a.sigmoid_scale * (ub / (float)a.HW);
      dp = a.dice_scale * (psum / (psum + a.smooth));
    }
    float* rs = a.rowstat + row * 8;
    rs[0] = S;
    rs[1] = P;
    rs[2] = mp;
    rs[3] = dp;
    rs[4] = pen;
  }
}
// ---------------------------------------------------------------------------
// wave64 helpers: DPP lane exchanges and a min-reduction without LDS traffic
// ---------------------------------------------------------------------------
// DPP move of one float64 with no initial value: the callers use only the
// lanes that the control word writes.
template <int CTRL, int ROWS>
__device__ __forceinline__ double mov_dpp_d(double v) {
  const uint64_t u = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)u, CTRL, ROWS, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(u >> 32), CTRL, ROWS, 0xF, false);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ double readlane_d(double v, int lane) {
  const uint64_t u = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
// The high word of a float64, and a float64 with its high word replaced.
__device__ __forceinline__ uint32_t hi_word(double x) {
  return (uint32_t)((uint64_t)__double_as_longlong(x) >> 32);
}
__device__ __forceinline__ double with_hi(double x, uint32_t hi) {
  const uint64_t u = (uint64_t)__double_as_longlong(x);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | (uint32_t)u));
}
// v_min_f64 as the hardware does it in IEEE mode (the kernels' mode): a quiet
// NaN operand yields the other operand.  Written out so that the compiler
// adds no canonicalising instructions around it.
__device__ __forceinline__ double min_f64(double a, double b) {
  double r;
  asm("v_min_f64 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
// Minimum of v over the wave (quiet NaNs ignored), wave-uniform: four DPP
// levels within each row of 16 lanes, then row_bcast:15 into rows 1 and 3
// and row_bcast:31 into rows 2 and 3 leave the wave's minimum in lane 63.
__device__ __forceinline__ double wave_min_f64(double v) {
  v = min_f64(v, mov_dpp_d<0xB1, 0xF>(v));   // quad_perm [1,0,3,2]
  v = min_f64(v, mov_dpp_d<0x4E, 0xF>(v));   // quad_perm [2,3,0,1]
  v = min_f64(v, mov_dpp_d<0x141, 0xF>(v));  // row_half_mirror
  v = min_f64(v, mov_dpp_d<0x140, 0xF>(v));  // row_mirror
  v = min_f64(v, mov_dpp_d<0x142, 0xA>(v));  // row_bcast:15
  v = min_f64(v, mov_dpp_d<0x143, 0xC>(v));  // row_bcast:31
  return readlane_d(v, 63);
}
// Index of the lowest set bit of a wave-uniform 64-bit lane mask, -1 (all
// ones) when the mask is empty: s_ff1_i32_b64 itself.
__device__ __forceinline__ uint32_t first_lane_s(uint64_t m) {
  uint32_t r;
  asm("s_ff1_i32_b64 %0, %1" : "=s"(r) : "s"(m) : "scc");
  return r;
}
// Scalar unsigned minimum and exponent bits of wave-uniform values (kept on
// the scalar unit: the compiler would otherwise move them to vector ops and
// read the result back).
__device__ __forceinline__ uint32_t min_s(uint32_t a, uint32_t b) {
  uint32_t r;
  asm("s_min_u32 %0, %1, %2" : "=s"(r) : "s"(a), "s"(b) : "scc");
  return r;
}
__device__ __forceinline__ uint32_t exp_bits_s(double x) {
  uint32_t r;
  asm("s_and_b32 %0, %1, 0x7ff00000" : "=s"(r) : "s"(hi_word(x)) : "scc");
  return r;
}
// The solver's per-slot state that is read or written at a wave-uniform slot
// (matched rows, their potentials, the predecessors) as vectors: the
// compiler then accesses slot t with VGPR index mode (s_set_gpr_idx_on, one
// v_mov per dword, s_set_gpr_idx_off) instead of a compare-and-select chain
// over every slot.  It picks the index mode for vectors whose select chain
// would take more than 16 instructions, hence 16 ints and at least 8
// doubles whatever NJ; slots NJ and up are never touched.
typedef int SlotsI __attribute__((ext_vector_type(16)));
template <int NJ>
using SlotsD = double __attribute__((ext_vector_type(NJ <= 8 ? 8 : 16)));
// Slot t (wave-uniform) of x.
template <int NJ, class V>
__device__ __forceinline__ auto slot_at(const V& x, int t) {
  if constexpr (NJ == 1) return x[0];
  else return x[__builtin_amdgcn_readfirstlane(t)];
}
template <int NJ, class V, class E>
__device__ __forceinline__ void slot_set(V& x, int t, E e) {
  if constexpr (NJ == 1) x[0] = e;
  else x[__builtin_amdgcn_readfirstlane(t)] = e;
}

// ---------------------------------------------------------------------------
// e-maxx Hungarian on one wave.  Rows = hrows[0..M) (GT columns), columns =
// preds[0..n) (queries).  asg[k] = row index assigned to column k, or -1.
// Mirrors src/cpu/matching.cpp:95-186 operation by operation.
//
// Column j = 1 + lane + 64 t lives in lane `lane`, register slot t: its
// potential v, its matched row p (0 = free), and, for that row, the row
// potential u[p] and its cost-matrix row; the row being inserted keeps its
// potential and cost row in wave-uniform registers.  So the Dijkstra steps
// touch LDS only for the cost entries, and every potential update is a
// register operation.  A column in the tree (and an unused slot) holds a
// quiet NaN in minv: no relaxation updates it (cur < NaN is false), the
// minimum ignores it (v_min_f64) and no comparison with delta matches it,
// so the steps carry no separate "used" state.  delta is one float64 DPP
// minimum over the wave; the entering column is the lowest one whose minv
// equals delta (one ballot per slot, its lowest lane, the lowest slot): the
// reference's scan keeps the first of equal minima (strict '<',
// src/cpu/matching.cpp:146-149), and a column's index grows with its slot,
// then its lane.  The next cost row's reads are issued as soon as its
// column is known, before the potential updates.  Each potential receives
// the same float64 operations in the same order as in the reference (one
// += delta or -= delta per step; a column outside the tree adds delta x 0,
// which leaves the value, up to the sign of a zero, which no later
// comparison or sum can see), so the assignment is the reference's bit for
// bit.
// ---------------------------------------------------------------------------
// Cost rows of one image, [column][query] with row stride ldq: all in LDS,
// or all read in place from finalize's total-cost plane (L2).
// CM, a compile-time choice so that each read is a ds_read or a global load:
// kCostLds (every row in LDS) or kCostGlobal (none).
enum { kCostGlobal = 0, kCostLds = 1 };
typedef __attribute__((address_space(3))) const float lds_f32;     // LDS
typedef __attribute__((address_space(1))) const float global_f32;  // device memory
template <int CM>
struct CostRows {
  // address-space qualified, so that a row read is a ds_read or a global load
  // and never a flat load through a pointer chosen at run time
  const lds_f32* lds;
  const global_f32* glb;
  // kCostGlobal: the staging pass's float64 copies of the rows, [column][query]
  // with row stride ldq, the invalid cost already replaced by BIG
  const double* glb64;
  int ldq;  // c * ldq fits 31 bits: Q <= 1024, and the column arrays fit the LDS
  // one element (per-lane column)
  __device__ __forceinline__ float at(int64_t c, int64_t q) const {
    return CM == kCostLds ? lds[c * ldq + q] : glb[c * ldq + q];
  }
};

// The row of column col, at the slots' query indices: a ds_read row or an
// in-place global row.
// Row entries as the solver reads them: float32 from the LDS (the invalid
// cost replaced in each step), float64 c(i, j) for rows read in place.
template <int CM>
using RowElem = typename std::conditional<CM == kCostLds, float, double>::type;
template <int NJ, int CM>
__device__ __forceinline__ void read_cost_row(const CostRows<CM>& cost, int col,
                                              const int (&predj)[NJ], RowElem<CM> (&raw)[NJ]) {
  if constexpr (CM == kCostLds) {
    const lds_f32* crow = cost.lds + col * cost.ldq;
#pragma unroll
    for (int t = 0; t < NJ; ++t) raw[t] = crow[predj[t]];
  } else {
    // buffer loads over the image's rows: the row's byte offset is a scalar
    // operand and the lane's query offset a loop-invariant 32-bit register,
    // so a row read needs no per-lane address arithmetic (reads past the
    // rows return 0: the rows are [rows][ldq] doubles, rows < 256)
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)cost.glb64, (short)0, 256 * cost.ldq * 8, 0x00020000);
    const int rowoff = col * cost.ldq * 8;
#pragma unroll
    for (int t = 0; t < NJ; ++t) {
      const u32x2_t w = __builtin_amdgcn_raw_buffer_load_b64(rsrc, predj[t] * 8, rowoff, 0);
      raw[t] = __builtin_bit_cast(double, w);
    }
  }
}
// c(i, j) of the reference (src/cpu/matching.cpp:497-511): the cost, or BIG
// for an invalid one (the plane holds a NaN for every non-finite cost, so
// raw < thr is cost_ok(raw)); rows read in place carry it already.
template <int CM>
__device__ __forceinline__ double cij_of(RowElem<CM> raw, double thr, double BIG) {
  if constexpr (CM == kCostLds) {
    const double r = (double)raw;
    return r < thr ? r : BIG;
  } else {
    return raw;
  }
}

// thr: the cost threshold.  The cost plane holds a NaN for every non-finite
// cost (finalize_kernel), so `raw < thr` is cost_ok(raw).
template <int NJ, int CM>
__device__ bool hungarian_wave(const CostRows<CM>& cost, const int* preds, int n,
                               const int* hrows, int M, double thr, double BIG, int* p, int* way,
                               double* u, int* asg) {
  (void)p;
  (void)way;
  (void)u;
  const int lane = threadIdx.x & 63;
  for (int k = lane; k < n; k += 64) asg[k] = -1;
  wave_sync();
  if (M == 0 || n == 0 || n < M) return true;
  const double kQNaN = __longlong_as_double(0x7FF8000000000000ll);
  double v[NJ];
  SlotsD<NJ> ucol = {};
  // pr: the column's matched row p (0 = free) in the low 16 bits and that
  // row's cost-matrix row in the high 16 (rows <= 1024, columns <= 256)
  SlotsI pr = {};
  int predj[NJ];
  bool valid[NJ];
#pragma unroll
  for (int t = 0; t < NJ; ++t) {
    const int j = 1 + lane + 64 * t;
    valid[t] = j <= n;
    v[t] = 0.0;
    ucol[t] = 0.0;
    pr[t] = 0;
    predj[t] = valid[t] ? preds[j - 1] : 0;
  }
  bool ok = true;
  // the cost row of the row being inserted is read before that row starts:
  // the first row's here, every later one's during the previous row's
  // augmentation walk, whose latency then hides the read
  int colcur = __builtin_amdgcn_readfirstlane(hrows[0]);
  RowElem<CM> rawf[NJ];
  read_cost_row<NJ, CM>(cost, colcur, predj, rawf);
  for (int i = 1; i <= M && ok; ++i) {
    const int colnext = i < M ? hrows[i] : colcur;  // no dependence: loaded early
    // minv: a quiet NaN marks a column in the tree (and an unused slot);
    // f: 1.0 for a column in the tree, else 0.0 (its low word stays 0)
    double minv[NJ], f[NJ];
    SlotsI wy = {};
#pragma unroll
    for (int t = 0; t < NJ; ++t) {
      minv[t] = valid[t] ? INFINITY : kQNaN;
      f[t] = 0.0;
      wy[t] = 0;
    }
    double ucur = 0.0;  // potential of row i (column 0 of the reference)
    int j0 = 0;
    double ui0 = ucur;
    for (;;) {
      // relax every column outside the tree (no branches: the NJ chains
      // interleave) and keep this lane's minimum
      double lm[NJ];
#pragma unroll
      for (int t = 0; t < NJ; ++t) {
        const double cij = cij_of<CM>(rawf[t], thr, BIG);
        const double cur = cij - ui0 - v[t];
        const bool upd = cur < minv[t];
        minv[t] = upd ? cur : minv[t];
        wy[t] = upd ? j0 : wy[t];
        lm[t] = minv[t];
      }
      // the lane's minimum as a tree (a lane whose slots all hold the NaN
      // marker gives NaN, which the wave minimum ignores like the markers)
#pragma unroll
      for (int w = 1; w < NJ; w *= 2)
#pragma unroll
        for (int t = 0; t + w < NJ; t += 2 * w) lm[t] = min_f64(lm[t], lm[t + w]);
      const double delta = wave_min_f64(lm[0]);
      // !(delta < inf), tested on the scalar high word: delta is +inf or a
      // NaN (no column left, unreachable with finite costs and n >= M free
      // columns); it is never -inf
      if (exp_bits_s(delta) == 0x7FF00000u) {
        ok = false;
        break;
      }
      // key = j1 - 1 of the entering column: the lowest (slot, lane) whose
      // minv equals delta, the minimum over the slots of the first lane of
      // each slot's ballot (an empty ballot gives all ones)
      // (every ballot is issued before the first scan, so the compares do
      // not wait for each other's mask registers)
      uint64_t bal[NJ];
#pragma unroll
      for (int t = 0; t < NJ; ++t) bal[t] = __builtin_amdgcn_ballot_w64(minv[t] == delta);
      __builtin_amdgcn_sched_barrier(0);
      uint32_t key = first_lane_s(bal[0]);
#pragma unroll
      for (int t = 1; t < NJ; ++t) key = min_s(key, first_lane_s(bal[t]) | (uint32_t)(64 * t));
      // potentials: columns in the tree (and column 0 = row i) move by delta
      // (f = 1), the others' minv by -delta; then column j1 enters the tree
#pragma unroll
      for (int t = 0; t < NJ; ++t) {
        ucol[t] = __builtin_fma(delta, f[t], ucol[t]);
        v[t] = __builtin_fma(-delta, f[t], v[t]);
        const bool enter = lane + 64 * t == (int)key;
        minv[t] = with_hi(minv[t] - delta, enter ? 0x7FF80000u : hi_word(minv[t] - delta));
        f[t] = with_hi(f[t], enter ? 0x3FF00000u : hi_word(f[t]));
      }
      ucur += delta;
      j0 = (int)key + 1;
      const int ol = (int)(key & 63u), ot = (int)(key >> 6);
      const int pr1 = __builtin_amdgcn_readlane(slot_at<NJ>(pr, ot), ol);
      if ((pr1 & 0xFFFF) == 0) break;  // j1 is free: augment
      // next row of the tree: the one matched to column j1 (its potential
      // took no delta above: j1 was outside the tree)
      ui0 = readlane_d(slot_at<NJ>(ucol, ot), ol);
      read_cost_row<NJ, CM>(cost, pr1 >> 16, predj, rawf);
    }
    if (!ok) break;
    const int cn = __builtin_amdgcn_readfirstlane(colnext);
    if (i < M) read_cost_row<NJ, CM>(cost, cn, predj, rawf);  // row i + 1's first step
    // augment along way[] from the free column j0 back to column 0: each
    // column on the path takes the row (and that row's potential and cost
    // row) of the column it was reached from; column 0 holds row i.
    for (int steps = 0; j0 != 0 && steps <= n; ++steps) {
      const int ol = (j0 - 1) & 63, ot = (j0 - 1) >> 6;
      const int jp = __builtin_amdgcn_readlane(slot_at<NJ>(wy, ot), ol);
      int npr;
      double nu;
      if (jp == 0) {
        npr = i | (colcur << 16);
        nu = ucur;
      } else {
        const int pl = (jp - 1) & 63, pt = (jp - 1) >> 6;
        npr = __builtin_amdgcn_readlane(slot_at<NJ>(pr, pt), pl);
        nu = readlane_d(slot_at<NJ>(ucol, pt), pl);
      }
      // the slot's old values read by every lane (kept unconditional, so the
      // new slot is one select, not an exec-masked read)
      int opr = slot_at<NJ>(pr, ot);
      double ou = slot_at<NJ>(ucol, ot);
      asm("" : "+v"(opr), "+v"(ou));
      const bool me = lane == ol;
      slot_set<NJ>(pr, ot, me ? npr : opr);
      slot_set<NJ>(ucol, ot, me ? nu : ou);
      j0 = jp;
    }
    colcur = cn;
  }
  if (ok) {
#pragma unroll
    for (int t = 0; t < NJ; ++t)
      if (valid[t] && (pr[t] & 0xFFFF) > 0) asg[lane + 64 * t] = (pr[t] & 0xFFFF) - 1;
  }
  wave_sync();
  return ok;
}

// Greedy over preds[0..n) with per-column capacities (src/cpu/matching.cpp:193-229).
// Column order = vcols[0..nv); ties -> earlier column (strict '<').
template <int CM>
__device__ void greedy_wave(const CostRows<CM>& cost, const int* preds, int n,
                            const int* vcols, int nv, int* cap, int* p2g, double thr) {
  const int lane = threadIdx.x & 63;
  for (int k = 0; k < n; ++k) {
    const int q = preds[k];
    if (p2g[q] >= 0) continue;
    double best = INFINITY;
    int bidx = 1 << 30;
    for (int t = lane; t < nv; t += 64) {
      const int c = vcols[t];
      if (cap[c] <= 0) continue;
      const double cv = (double)cost.at(c, q);
      if (!cost_ok(cv, thr)) continue;
      if (cv < best) {
        best = cv;
        bidx = t;
      }
    }
    const double m = wave_min_d(best);
    int pick = -1;
    if (m < INFINITY) {
      const uint64_t hit = __ballot(best == m);
      // lowest column index t among lanes attaining m
      int cand = best == m ? bidx : (1 << 30);
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) cand = min(cand, __shfl_xor(cand, o, 64));
      (void)hit;
      pick = vcols[cand];
    }
    if (lane == 0 && pick >= 0) {
      p2g[q] = pick;
      if (cap[pick] > 0) cap[pick] -= 1;
    }
    wave_sync();
  }
}

// Per-layer means and denominators (src/cuda/mask_matching_forward.cu:549-583),
// then, with a saved state, the list of matched query rows in ascending order
// (wave ballots, one blockDim-row chunk at a time) for the backward.  One
// workgroup.
__device__ void layer_pass(const LayerArgs& a, int* sbuf, int nsbuf) {
  for (int64_t l = threadIdx.x; l < a.L; l += blockDim.x) {
    float m = 0.f, d = 0.f, c = 0.f, cnt = 0.f;
    for (int64_t b = 0; b < a.B; ++b) {
      const float* s = a.img + (l * a.B + b) * 4;
      m += s[0];
      d += s[1];
      c += s[2];
      cnt += s[3];
    }
    const float total = (float)(a.B * a.Q);
    const bool has_nm = a.num_masks > 0.0;
    float md = a.force_masks ? total : (has_nm ? (float)a.num_masks : cnt);
    float cd = (a.force_cls || a.has_void) ? total : (has_nm ? (float)a.num_masks : cnt);
    md = fmaxf(md, 1.f);
    cd = fmaxf(cd, 1.f);
    a.means[0 * a.L + l] = m / md;
    a.means[1 * a.L + l] = d / md;
    a.means[2 * a.L + l] = c / cd;
    a.layer[l * ML_LAYERS + ML_LAYER_INV_MASK_DEN] = 1.f / md;
    a.layer[l * ML_LAYERS + ML_LAYER_INV_CLS_DEN] = 1.f / cd;
  }
  if (a.list == nullptr) return;
  // the matched-row list: the slices' own lists (mrows, written by their
  // assignment workgroups) concatenated in slice order, i.e. ascending row
  // index; slices in chunks of CH (prefix and count of each in sbuf), each
  // chunk one block scan of the counts and one flattened copy
  __shared__ int wtot[16];
  const int tid = threadIdx.x, nt = blockDim.x;
  const int wave = tid >> 6, lane = tid & 63, nw = nt >> 6;
  const int64_t LB = a.L * a.B;
  const int CH = min(nt, nsbuf / 2);
  int base = 0;
  for (int64_t c0 = 0; c0 < LB; c0 += CH) {
    const int nc = (int)min((int64_t)CH, LB - c0);
    const int cnt = tid < nc ? (int)a.img[(c0 + tid) * 4 + 3] : 0;
    int incl = cnt;  // inclusive scan within the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(incl, o, 64);
      incl += lane >= o ? y : 0;
    }
    if (lane == 63) wtot[wave] = incl;
    __syncthreads();
    int before = 0, total = 0;
    for (int w = 0; w < nw; ++w) {
      before += w < wave ? wtot[w] : 0;
      total += wtot[w];
    }
    if (tid < nc) {
      sbuf[tid] = before + incl - cnt;  // exclusive prefix within the chunk
      sbuf[CH + tid] = cnt;
    }
    __syncthreads();
    for (int g = tid; g < total; g += nt) {
      // the last slice whose prefix is <= g holds output g
      int lo = 0, hi = nc - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (sbuf[mid] <= g) lo = mid;
        else hi = mid - 1;
      }
      a.list[1 + base + g] = a.mrows[(c0 + lo) * a.Q + (g - sbuf[lo])];
    }
    base += total;
    __syncthreads();  // sbuf and wtot are reused by the next chunk
  }
  if (tid == 0) a.list[0] = base;
}

// CM: where the image's cost rows live (CostRows): all in LDS when the
// matrix fits, else read in place from finalize's total-cost plane.
// Workgroups L*B .. L*B + fill_blocks - 1 zero-fill the gradient buffer:
// the assignment keeps one CU per image busy with a serial chain and leaves
// HBM idle, so the fill runs beside it in the same launch, from its start
// (the fill's writes slow the images' row staging a little, which the
// solvers' slack absorbs: measured 7 us shorter than a fill that waits for
// the staging).

// Copy the cost rows of image b's non-empty GT columns (colmap order) from
// finalize's plane into LDS (kCostLds) or, as float64 c(i, j) with BIG for an
// invalid cost, into tot64 (kCostGlobal), and mark the valid columns (one cost
// finite and below the threshold, cost_ok).  One wave per row, V floats per
// load (V = 4 when rows start on 16-byte boundaries), R rows per wave in
// flight; Q <= 64 * NJ, so a lane holds at most KW words of a row.
template <int V, int NJ, int CM>
__device__ __forceinline__ void stage_rows(const AssignArgs& a, int64_t lb, int64_t b,
                                           float* costL, int64_t lds_rows, int* colok) {
  typedef typename std::conditional<V == 4, float4, float>::type word_t;
  constexpr int KW = V == 4 ? (NJ + 3) / 4 : NJ;
  constexpr int R = KW == 1 ? 8 : KW == 2 ? 4 : 2;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int G = __builtin_amdgcn_readfirstlane(a.ncols[b]);
  const int* cm = a.colmap + b * a.nslot;
  const int W = (int)(a.Q / V);  // words per row
  const word_t* src = (const word_t*)(a.tot + lb * a.tot_stride);
  for (int s0 = wave * R; s0 < G; s0 += 4 * R) {
    word_t v[R][KW];
    int col[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      col[r] = s0 + r < G ? cm[s0 + r] : -1;
#pragma unroll
      for (int k = 0; k < KW; ++k) {
        const int j = lane + 64 * k;
        if (col[r] >= 0 && j < W) v[r][k] = src[(int64_t)col[r] * W + j];
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (col[r] < 0) continue;  // wave-uniform
      bool ok = false;
#pragma unroll
      for (int k = 0; k < KW; ++k) {
        const int j = lane + 64 * k;
        if (j >= W) continue;
        if (CM == kCostLds)
          ((word_t*)costL)[(int64_t)col[r] * W + j] = v[r][k];
        const float* e = (const float*)&v[r][k];
        double c64[V];
#pragma unroll
        for (int h = 0; h < V; ++h) {
          const bool okh = cost_ok((double)e[h], a.inf_thresh);
          ok |= okh;
          c64[h] = okh ? (double)e[h] : a.big;
        }
        if (CM == kCostGlobal) {
          double* dst = a.tot64 + (lb * a.GT_out + col[r]) * a.Q + (int64_t)j * V;
#pragma unroll
          for (int h = 0; h < V; ++h) dst[h] = c64[h];
        }
      }
      if (__ballot(ok) != 0ull && lane == 0) colok[col[r]] = 1;
    }
  }
}

template <int NJ, int CM>
__global__ __launch_bounds__(256) void assign_kernel(AssignArgs a) {
  if ((int64_t)blockIdx.x >= a.L * a.B) {
    zero_fill_range(a.fill, a.fill_n16, a.fill_tail, a.fill_ntail,
                    (int64_t)blockIdx.x - a.L * a.B, a.fill_blocks);
    return;
  }
  extern __shared__ __align__(16) unsigned char smem[];
  const SmemLayout L = smem_layout(a.Q, a.GT_out, CM == kCostGlobal ? 0 : a.lds_rows);
  float* contrib = (float*)(smem + L.contrib);
  int* colok = (int*)(smem + L.colok);
  int* vcols = (int*)(smem + L.vcols);
  int* preds = (int*)(smem + L.preds);
  int* pp = (int*)(smem + L.p);
  int* way = (int*)(smem + L.way);
  double* u = (double*)(smem + L.u);
  int* hrows = (int*)(smem + L.hrows);
  int* asg = (int*)(smem + L.asg);

  // A serial, latency-bound chain: take issue priority over waves of the
  // fill workgroups should they share the CU.
  __builtin_amdgcn_s_setprio(3);
  const int64_t lb = blockIdx.x, b = lb % a.B;
  // another launch's image: no work, no count (the column count is read only
  // for a launch restricted to a subset)
  if (a.phase_class >= 0 &&
      !in_phase(a.phase_class, a.phase_in, __builtin_amdgcn_readfirstlane(a.ncols[b])))
    return;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t Q = a.Q, GTo = a.GT_out;
  float* costL = (float*)(smem + L.costL);
  CostRows<CM> crows;
  crows.lds = (const lds_f32*)costL;
  crows.glb = (const global_f32*)(a.tot + lb * a.tot_stride);
  crows.glb64 = CM == kCostGlobal ? a.tot64 + lb * a.GT_out * a.Q : nullptr;
  crows.ldq = (int)Q;
  const int64_t term = a.L * a.B * Q * GTo;
  const float* sep = a.sep + lb * Q * GTo;

  // ---- 1. the image's total cost (bce + dice) + cls (src/cpu/matching.cpp:665),
  //         [column][query] from finalize, into LDS; column validity
  //         (matching.cpp:497-511).  Only the rows of non-empty GTs are
  //         staged: an empty GT's costs are +inf, so its column is invalid
  //         and its row is never read.
  for (int64_t c = tid; c <= GTo; c += 256) colok[c] = 0;
  __syncthreads();
  if ((Q & 3) == 0) stage_rows<4, NJ, CM>(a, lb, b, costL, a.lds_rows, colok);
  else stage_rows<1, NJ, CM>(a, lb, b, costL, a.lds_rows, colok);
  __syncthreads();

  // ---- 2. assignment on wave 0
  if (wave == 0) {
    int nv = 0;
    for (int64_t c0 = 0; c0 < GTo; c0 += 64) {
      const int64_t c = c0 + lane;
      const bool okc = c < GTo && colok[c];
      const uint64_t m = __ballot(okc);
      if (okc) vcols[nv + __popcll(m & ((1ull << lane) - 1ull))] = (int)c;
      nv += __popcll(m);
    }
    int* p2g = asg;         // per-query result (-1 or column)
    int* hout = (int*)contrib;  // output of one Hungarian call
    for (int64_t q = lane; q < Q; q += 64) p2g[q] = -1;
    wave_sync();
    const double thr = a.inf_thresh, BIG = a.big;
    const int64_t K = a.topk;
    bool okh = true;
    if (Q > 0 && GTo > 0 && K > 0 && nv > 0) {
      int* cap = colok;  // capacities (column validity no longer needed)
      for (int64_t c = lane; c < GTo; c += 64) cap[c] = 0;
      wave_sync();
      for (int t = lane; t < nv; t += 64) cap[vcols[t]] = (int)K;
      for (int64_t q = lane; q < Q; q += 64) preds[q] = (int)q;
      wave_sync();
      if (a.strategy == ML_GLOBAL || a.strategy == ML_PSEUDO_GREEDY) {
        // the assignment's rows: the valid columns, repeated K times for
        // global (once for pseudo-greedy), at most Q of them
        const int64_t reps = a.strategy == ML_GLOBAL ? K : 1;
        const int M = (int)min(reps * (int64_t)nv, Q);
        for (int k = lane; k < M; k += 64) hrows[k] = vcols[k % nv];
        wave_sync();
        okh = hungarian_wave<NJ>(crows, preds, (int)Q, hrows, M, thr, BIG, pp, way, u, hout);
        if (okh) {
          for (int64_t q = lane; q < Q; q += 64) {
            const int r = hout[q];
            if (r >= 0) {
              const int c = hrows[r];
              if (cost_ok((double)crows.at(c, q), thr)) p2g[q] = c;
            }
          }
          wave_sync();
          if (a.strategy == ML_PSEUDO_GREEDY) {
            if (lane == 0)
              for (int64_t q = 0; q < Q; ++q)
                if (p2g[q] >= 0 && cap[p2g[q]] > 0) cap[p2g[q]] -= 1;
            wave_sync();
            int nr = 0;
            for (int64_t q0 = 0; q0 < Q; q0 += 64) {
              const int64_t q = q0 + lane;
              const bool un = q < Q && p2g[q] < 0;
              const uint64_t m = __ballot(un);
              if (un) preds[nr + __popcll(m & ((1ull << lane) - 1ull))] = (int)q;
              nr += __popcll(m);
            }
            wave_sync();
            if (nr > 0) greedy_wave(crows, preds, nr, vcols, nv, cap, p2g, thr);
          }
        }
      } else if (a.strategy == ML_ROUND) {
        int nrem = (int)Q;
        for (int64_t rd = 0; rd < K && okh; ++rd) {
          int M = 0;
          for (int t = 0; t < nv; ++t)
            if (cap[vcols[t]] > 0) {
              if (lane == 0) hrows[M] = vcols[t];
              ++M;
            }
          if (M == 0 || nrem == 0) break;
          if (M > nrem) M = nrem;
          wave_sync();
          okh = hungarian_wave<NJ>(crows, preds, nrem, hrows, M, thr, BIG, pp, way, u, hout);
          if (!okh) break;
          // apply in query order and compact the remaining queries (order kept)
          int nn = 0;
          for (int k0 = 0; k0 < nrem; k0 += 64) {
            const int k = k0 + lane;
            bool keep = false;
            int q = -1;
            if (k < nrem) {
              q = preds[k];
              const int r = hout[k];
              if (r >= 0) {
                const int c = hrows[r];
                if (!cost_ok((double)crows.at(c, q), thr)) keep = true;
                else p2g[q] = c;
              } else {
                keep = true;
              }
            }
            const uint64_t m = __ballot(keep);
            if (keep) way[nn + __popcll(m & ((1ull << lane) - 1ull))] = q;
            nn += __popcll(m);
          }
          wave_sync();
          if (lane == 0)
            for (int k = 0; k < nrem; ++k) {
              const int q = preds[k];
              const int c = p2g[q];
              if (c >= 0 && hout[k] >= 0 && hrows[hout[k]] == c && cap[c] > 0) cap[c] -= 1;
            }
          wave_sync();
          for (int k = lane; k < nn; k += 64) preds[k] = way[k];
          nrem = nn;
          wave_sync();
          if (nrem == 0) break;
        }
      } else if (a.strategy == ML_GREEDY) {
        greedy_wave(crows, preds, (int)Q, vcols, nv, cap, p2g, thr);
      }
    }
    if (!okh) {  // no finite augmenting path (invalid costs are BIG): image left unmatched
      for (int64_t q = lane; q < Q; q += 64) p2g[q] = -1;
    }
    // drop invalid, rank by (cost, q) within each column (matching.cpp:533-565)
    for (int64_t q = lane; q < Q; q += 64) {
      const int c = p2g[q];
      if (c >= 0 && !cost_ok((double)crows.at(c, q), thr)) p2g[q] = -1;
    }
    wave_sync();
    // compact the matched queries; rank each among those of its column
    int nm = 0;
    int* mq = preds;  // matched query list (preds no longer needed)
    for (int64_t q0 = 0; q0 < Q; q0 += 64) {
      const int64_t q = q0 + lane;
      const bool mt = q < Q && p2g[q] >= 0;
      const uint64_t m = __ballot(mt);
      if (mt) mq[nm + __popcll(m & ((1ull << lane) - 1ull))] = (int)q;
      nm += __popcll(m);
    }
    wave_sync();
    if (a.layer_args.list) {  // this slice's part of the saved matched-row list
      int* mr = a.layer_args.mrows + lb * Q;
      for (int k = lane; k < nm; k += 64) mr[k] = (int)(lb * Q + mq[k]);
    }
    for (int64_t q = lane; q < Q; q += 64) {
      const int c = p2g[q];
      int64_t rnd = -1;
      if (c >= 0) {
        int64_t rank = 0;
        if (K > 1) {
          const float cq = crows.at(c, q);
          for (int k = 0; k < nm; ++k) {
            const int q2 = mq[k];
            if (q2 == q || p2g[q2] != c) continue;
            const float c2 = crows.at(c, q2);
            if (c2 < cq || (c2 == cq && q2 < q)) ++rank;
          }
        }
        rnd = rank < K ? rank : -1;
      }
      a.pred_to_gt[lb * Q + q] = c;
      a.pred_round[lb * Q + q] = rnd;
    }
  }
  __syncthreads();

  // ---- 3. matched-loss partial sums and backward statistics
  const int* p2g = asg;
  const bool need_cls_pen = a.force_cls || a.void_idx >= 0;
  for (int64_t q = tid; q < Q; q += 256) {
    const int c = p2g[q];
    const float* rs = a.rowstat + (lb * Q + q) * 8;
    float cm = 0.f, cd = 0.f, cc = 0.f, I = 0.f, T = 0.f;
    if (c >= 0) {
      cm = sep[q * GTo + c];
      cd = sep[term + q * GTo + c];
      cc = sep[2 * term + q * GTo + c];
      const int slot = a.slot_of_col[b * GTo + c];
      if (slot >= 0 && a.rowIT) {
        const float2 it = ((const float2*)a.rowIT)[(lb * Q + q) * a.nslot + slot];
        I = it.x;
        T = it.y;
      }
    } else {
      if (a.force_masks) {
        cm = rs[2];
        cd = rs[3];
      }
      if (need_cls_pen) cc = rs[4];
    }
    contrib[q * 4 + 0] = cm;
    contrib[q * 4 + 1] = cd;
    contrib[q * 4 + 2] = cc;
    contrib[q * 4 + 3] = c >= 0 ? 1.f : 0.f;
    if (a.stats) {
      float* st = a.stats + (lb * Q + q) * ML_STATS;
      st[ML_STAT_S] = rs[0];
      st[ML_STAT_P] = rs[1];
      st[ML_STAT_I] = I;
      st[ML_STAT_T] = T;
    }
  }
  __syncthreads();
  if (wave == 0) {
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    for (int64_t q = lane; q < Q; q += 64) {
      s0 += contrib[q * 4 + 0];
      s1 += contrib[q * 4 + 1];
      s2 += contrib[q * 4 + 2];
      s3 += contrib[q * 4 + 3];
    }
    s0 = wave_sum(s0);
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    s3 = wave_sum(s3);
    if (lane == 0) {
      a.img[lb * 4 + 0] = s0;
      a.img[lb * 4 + 1] = s1;
      a.img[lb * 4 + 2] = s2;
      a.img[lb * 4 + 3] = s3;
    }
  }
  // ---- 4. the last image to finish runs the per-layer pass (means,
  //         denominators, matched-row list) over every image's results:
  //         release this workgroup's writes, count it, and acquire the others'
  if (a.done) {
    __shared__ int last;
    __syncthreads();
    if (tid == 0) {
      __threadfence();
      last = atomicAdd(a.done, 1) == (int)(a.L * a.B) - 1;
      __threadfence();
    }
    __syncthreads();
    if (last) layer_pass(a.layer_args, (int*)smem, (int)(L.total / 4));
  }
}


__global__ __launch_bounds__(1024) void layer_kernel(LayerArgs a) {
  __shared__ int sbuf[2048];
  layer_pass(a, sbuf, 2048);
}

// Denominators from pred_to_gt alone (backward without saved statistics,
// src/cuda/mask_matching_backward.cu:480-508).  One wave per layer.
__global__ void layer_from_p2g_kernel(const int64_t* p2g, float* layer, int64_t L, int64_t B,
                                      int64_t Q, double num_masks, int force_masks,
                                      int force_cls, int has_void) {
  const int64_t l = blockIdx.x;
  const int lane = threadIdx.x;
  float cnt = 0.f;
  for (int64_t i = lane; i < B * Q; i += 64) cnt += p2g[l * B * Q + i] >= 0 ? 1.f : 0.f;
  cnt = wave_sum(cnt);
  if (lane == 0) {
    const float total = (float)(B * Q);
    const bool has_nm = num_masks > 0.0;
    float md = force_masks ? total : (has_nm ? (float)num_masks : cnt);
    float cd = (force_cls || has_void) ? total : (has_nm ? (float)num_masks : cnt);
    layer[l * ML_LAYERS + ML_LAYER_INV_MASK_DEN] = 1.f / fmaxf(md, 1.f);
    layer[l * ML_LAYERS + ML_LAYER_INV_CLS_DEN] = 1.f / fmaxf(cd, 1.f);
  }
}

size_t assign_smem_bytes(int64_t Q, int64_t GTo, int64_t lds_rows) {
  return smem_layout(Q, GTo, lds_rows).total;
}

template <int NJ, int CM>
static int launch_nj_l(const AssignArgs& a, const Dims& d, hipStream_t st, const char* prof) {
  const size_t sm = smem_layout(a.Q, a.GT_out, CM == kCostGlobal ? 0 : a.lds_rows).total;
  // 160 KB of LDS less the kernel's static part, raised once per device (the
  // attribute is set with that device current); the lock makes the first
  // call of several host threads safe
  constexpr int kMaxDev = 64;
  static std::atomic<size_t> max_dyn[kMaxDev];
  static std::mutex mu;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev)
    return fail(ML_ELAUNCH, "assign: no current device (or more than 64)");
  if (max_dyn[dev].load(std::memory_order_acquire) == 0) {
    std::lock_guard<std::mutex> g(mu);
    if (max_dyn[dev].load(std::memory_order_relaxed) == 0) {
      hipFuncAttributes fa;
      if (hipFuncGetAttributes(&fa, (const void*)assign_kernel<NJ, CM>) != hipSuccess)
        return fail(ML_ELAUNCH, "assign: cannot query the kernel attributes");
      const size_t dyn = 160 * 1024 - fa.sharedSizeBytes;
      if (hipFuncSetAttribute((const void*)assign_kernel<NJ, CM>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)dyn) != hipSuccess)
        return fail(ML_ELAUNCH, "assign: cannot raise the LDS limit");
      max_dyn[dev].store(dyn, std::memory_order_release);
    }
  }
  const size_t max_dyn_dev = max_dyn[dev].load(std::memory_order_acquire);
  if (sm > max_dyn_dev) return fail(ML_EUNSUPPORTED, "assign: cost matrix exceeds the LDS budget");
  {
    ProfScope ps_(prof, st);
    hipLaunchKernelGGL((assign_kernel<NJ, CM>), dim3((unsigned)(d.LB + a.fill_blocks)),
                       dim3(256), sm, st, a);
  }
  return check_launch("assign");
}
template <int NJ>
static int launch_nj(const AssignArgs& a, const Dims& d, hipStream_t st, const char* prof) {
  if (a.lds_rows >= a.GT_out) return launch_nj_l<NJ, kCostLds>(a, d, st, prof);
  return launch_nj_l<NJ, kCostGlobal>(a, d, st, prof);
}
int launch_finalize(const AssignArgs& a, const Dims& d, hipStream_t st, const char* prof) {
  const int64_t rows = d.LB * d.Q;
  if (rows == 0) return ML_OK;
  if (rows >= ((int64_t)1 << 31)) return fail(ML_EINVAL, "L * B * Q must be below 2^31");
  ProfScope ps_(prof, st);
  const dim3 grid((unsigned)(ceil_div(rows, 4) + a.fin_fill.blocks));
  const bool fast = a.cls_logits && a.C >= 1 && a.C <= 64 * kFinCls && a.GT_out >= 1 &&
                    a.GT_out <= 64 * kFinCols;
  const bool wide = !fast && a.cls_logits && a.C >= 1 && a.GT_out >= 1 && a.GT_out <= 64 * kFinColsWide;
  const bool wide_regs = wide && a.C <= 64 * kFinClsWide;
  const int dt = a.cls_logits ? a.cls_dtype : ML_BF16;
  if (wide_regs) {
    constexpr int NC = kFinClsWide, NG = kFinColsWide;
    if (dt == ML_F32) hipLaunchKernelGGL((finalize_kernel<ML_F32, true, NC, NG>), grid, dim3(256), 0, st, a);
    else if (dt == ML_F16) hipLaunchKernelGGL((finalize_kernel<ML_F16, true, NC, NG>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((finalize_kernel<ML_BF16, true, NC, NG>), grid, dim3(256), 0, st, a);
  } else if (fast) {
    if (dt == ML_F32) hipLaunchKernelGGL((finalize_kernel<ML_F32, true>), grid, dim3(256), 0, st, a);
    else if (dt == ML_F16) hipLaunchKernelGGL((finalize_kernel<ML_F16, true>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((finalize_kernel<ML_BF16, true>), grid, dim3(256), 0, st, a);
  } else if (wide) {
    constexpr int NC = 0, NG = kFinColsWide;
    if (dt == ML_F32) hipLaunchKernelGGL((finalize_kernel<ML_F32, true, NC, NG>), grid, dim3(256), 0, st, a);
    else if (dt == ML_F16) hipLaunchKernelGGL((finalize_kernel<ML_F16, true, NC, NG>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((finalize_kernel<ML_BF16, true, NC, NG>), grid, dim3(256), 0, st, a);
  } else {
    if (dt == ML_F32) hipLaunchKernelGGL((finalize_kernel<ML_F32, false>), grid, dim3(256), 0, st, a);
    else if (dt == ML_F16) hipLaunchKernelGGL((finalize_kernel<ML_F16, false>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((finalize_kernel<ML_BF16, false>), grid, dim3(256), 0, st, a);
  }
  return check_launch("finalize");
}

int launch_assign(const AssignArgs& a, const Dims& d, hipStream_t st, const char* prof) {
  const int64_t nj = ceil_div(a.Q, 64);
  // one instance per column count up to 6 per lane: the Dijkstra step's work
  // is proportional to NJ
  if (nj <= 1) return launch_nj<1>(a, d, st, prof);
  if (nj <= 2) return launch_nj<2>(a, d, st, prof);
  if (nj <= 3) return launch_nj<3>(a, d, st, prof);
  if (nj <= 4) return launch_nj<4>(a, d, st, prof);
  if (nj <= 5) return launch_nj<5>(a, d, st, prof);
  if (nj <= 6) return launch_nj<6>(a, d, st, prof);
  if (nj <= 8) return launch_nj<8>(a, d, st, prof);
  if (nj <= 16) return launch_nj<16>(a, d, st, prof);
  return fail(ML_EUNSUPPORTED, "more than 1024 queries per image are not supported");
}

int launch_layer(const LayerArgs& a, hipStream_t st) {
  {
    ProfScope ps_("layer", st);
    hipLaunchKernelGGL(layer_kernel, dim3(1), dim3(1024), 0, st, a);
  }
  return check_launch("layer");
}

int launch_layer_from_p2g(const int64_t* p2g, float* layer, int64_t L, int64_t B, int64_t Q,
                          double num_masks, int force_masks, int force_cls, int has_void,
                          hipStream_t st) {
  hipLaunchKernelGGL(layer_from_p2g_kernel, dim3((unsigned)L), dim3(64), 0, st, p2g, layer, L, B,
                     Q, num_masks, force_masks, force_cls, has_void);
  return check_launch("layer_from_p2g");
}

}  // namespace ml
