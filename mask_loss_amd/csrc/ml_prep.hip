// Target preparation: int64 label map -> compact per-image target operands.
//
//   s == 1 : u16 label per cell (labels outside [0, GT_total) -> 0xFFFF)
//   s  > 1 : count of each label inside the s x s block of every cell
//            (B, GT_total, HWp), the reference's count tensor
//            (src/cuda/utils.cuh:6-36); u8 for s <= 15, u16 for s >= 16
//            (where the reference's uint8 counts overflow, utils.cuh:9)
// plus, for the forward, which GTs have pixels (the reference's per-GT areas
// of src/cuda/pw_mask.cu:391 are only ever tested against zero) and, per
// image, the compacted list of output columns whose GT is non-empty, and the
// cost schedule.
#include "ml_internal.h"

namespace ml {

__global__ void fill_u32_kernel(uint32_t* p, uint32_t v, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) p[i] = v;
}

int launch_fill_i32(int* p, int v, int64_t n, hipStream_t st) {
  if (n <= 0) return ML_OK;
  int64_t blocks = ceil_div(n, 256);
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)blocks), dim3(256), 0, st, (uint32_t*)p,
                     (uint32_t)v, n);
  return check_launch("fill");
}

__global__ __launch_bounds__(256) void zero_fill_kernel(u32x4_t* p, int64_t n16,
                                                        unsigned char* tail, int64_t ntail) {
  zero_fill_range(p, n16, tail, ntail, blockIdx.x, gridDim.x);
}

int launch_zero_fill(void* p, size_t bytes, hipStream_t st) {
  if (bytes == 0) return ML_OK;
  const int64_t n16 = (int64_t)(bytes / 16);
  const int64_t ntail = (int64_t)(bytes % 16);
  int64_t blocks = ceil_div(n16 > 0 ? n16 : 1, 256);
  if (blocks > kFillBlocks) blocks = kFillBlocks;
  hipLaunchKernelGGL(zero_fill_kernel, dim3((unsigned)blocks), dim3(256), 0, st, (u32x4_t*)p, n16,
                     (unsigned char*)p + n16 * 16, ntail);
  return check_launch("zero_fill");
}

// Read-only stream: workgroup g reads its contiguous chunk of the n16 16-byte
// words, eight loads in flight per thread, and writes one word (so that no
// load is dead code).
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4_t* p, int64_t n16, uint32_t* out) {
  const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const int64_t b0 = min(n16, (int64_t)blockIdx.x * per), b1 = min(n16, b0 + per);
  uint32_t acc = 0;
  int64_t i = b0 + threadIdx.x;
  for (; i + 7 * 256 < b1; i += 8 * 256) {
    u32x4_t v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = p[i + u * 256];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  for (; i < b1; i += 256) {
    const u32x4_t v = p[i];
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  __shared__ uint32_t s;
  if (threadIdx.x == 0) s = 0u;
  __syncthreads();
  atomicXor(&s, acc);
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = s;
}

int launch_stream_read(const void* p, int64_t n16, uint32_t* out, int grid, hipStream_t st) {
  hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)grid), dim3(256), 0, st, (const u32x4_t*)p, n16, out);
  return check_launch("stream_read");
}

// flag[0] = any(x[i] == value), one workgroup.
__global__ __launch_bounds__(256) void any_equal_kernel(const int64_t* x, int64_t n, int64_t value,
                                                        int32_t* flag) {
  int hit = 0;
  for (int64_t i = threadIdx.x; i < n; i += 256) hit |= x[i] == value;
  hit = __syncthreads_or(hit);
  if (threadIdx.x == 0) flag[0] = hit ? 1 : 0;
}

int launch_any_equal(const int64_t* x, int64_t n, int64_t value, int32_t* flag, hipStream_t st) {
  hipLaunchKernelGGL(any_equal_kernel, dim3(1), dim3(256), 0, st, x, n, value, flag);
  return check_launch("any_equal");
}

// Presence marks of one preparation workgroup: a label bit set in LDS (lanes
// of a wave that agree with lane 0 skip the atomic: most cells of a wave carry
// one label); at the end the workgroup writes all kPresWords words of its
// record, so the record never needs clearing.
__device__ __forceinline__ void pres_clear(uint32_t* pres) {
  if (threadIdx.x < kPresWords) pres[threadIdx.x] = 0u;
}
__device__ __forceinline__ void pres_mark(uint32_t* pres, int64_t lab) {
  atomicOr(&pres[lab >> 5], 1u << (lab & 31));
}
__device__ __forceinline__ void pres_store(const PrepArgs& a, const uint32_t* pres, int64_t b) {
  if (threadIdx.x < kPresWords)
    a.pbits[(b * a.nblk + blockIdx.x) * kPresWords + threadIdx.x] = pres[threadIdx.x];
}

// The void-class check of every image's class targets, made by a workgroup
// of its own (the preparation grid's extra column, blockIdx.x == nblk, image
// row 0) so that the word is written early in the forward's first kernel
// without delaying a preparation workgroup (a host may be polling it):
// *void_found = any(cls_targets == void_idx), 0 without a valid void index,
// stored with system scope (the word may be pinned host memory).
__device__ __forceinline__ void void_check(const PrepArgs& a) {
  int hit = 0;
  if (a.void_idx >= 0) {
    const int64_t n = a.B * a.GT_total;
    for (int64_t i0 = threadIdx.x; i0 < n; i0 += 8 * (int64_t)blockDim.x) {
      int64_t v[8];  // eight loads in flight per thread, then the compares
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int64_t i = i0 + k * (int64_t)blockDim.x;
        v[k] = i < n ? a.cls_targets[i] : -1;
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) hit |= v[k] == a.void_idx;
    }
  }
  hit = __syncthreads_or(hit);
  if (threadIdx.x == 0)
    __hip_atomic_store(a.void_found, hit ? 1 : 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

constexpr int kColsLds = 1024;

// Compacted list of the columns whose GT is non-empty, one wave per image
// (images w, w + nwaves, ...), then, on wave 0, the cost schedule (per
// column-tile class: its tasks in ascending order, their count and K-split;
// per task: its position in its class list).  Run by one workgroup after the
// target-preparation grid.  Column counts of up to kColsLds images stay in
// LDS for the schedule pass.
__device__ void columns_and_schedule(const PrepArgs& a) {
  __shared__ int ncols_s[kColsLds];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nw = blockDim.x >> 6;
  const uint64_t below = (1ull << lane) - 1ull;
  for (int64_t b = wave; b < a.B; b += nw) {
    // presence word j = OR over the image's preparation workgroups: lane
    // (k0, j) with j = lane & 7 ORs workgroups k0, k0 + 8, ..., then the
    // eight k0 lanes of each word combine
    const int j = lane & (kPresWords - 1);
    const uint32_t* rec = a.pbits + b * a.nblk * kPresWords + j;
    uint32_t pq[4] = {0u, 0u, 0u, 0u};  // four records in flight per lane
    int64_t k = lane >> 3;
    for (; k + 24 < a.nblk; k += 32) {
#pragma unroll
      for (int u = 0; u < 4; ++u) pq[u] |= rec[(k + 8 * u) * kPresWords];
    }
    for (; k < a.nblk; k += 8) pq[0] |= rec[k * kPresWords];
    uint32_t pw = (pq[0] | pq[1]) | (pq[2] | pq[3]);
    pw |= __shfl_xor(pw, 8, 64);
    pw |= __shfl_xor(pw, 16, 64);
    pw |= __shfl_xor(pw, 32, 64);
    int base = 0;
    for (int64_t c0 = 0; c0 < a.GT_out; c0 += 64) {
      const int64_t c = c0 + lane;
      const int64_t act = c + (c >= a.bg ? 1 : 0);
      // lanes 0..7 hold words 0..7; every lane takes part in the shuffle
      const uint32_t word = __shfl(pw, (int)((act >> 5) & (kPresWords - 1)), 64);
      const bool ok = c < a.GT_out && ((word >> (act & 31)) & 1u);
      const uint64_t m = __ballot(ok);
      const int slot = base + __popcll(m & below);
      if (c < a.GT_out) {
        a.slot_of_col[b * a.GT_out + c] = ok ? slot : -1;
        if (ok) a.colmap[b * a.nslot + slot] = (int)c;
      }
      base += __popcll(m);
    }
    for (int s = base + lane; s < a.nslot; s += 64) a.colmap[b * a.nslot + s] = -1;
    if (lane == 0) {
      a.ncols[b] = base;
      if (b < kColsLds) ncols_s[b] = base;
    }
  }
  if (!a.sched) return;
  __syncthreads();
  if (wave != 0) return;
  const int64_t nt = a.plan.ntasks;
  int* list = a.sched + kSchedList;
  int* idx = list + kClasses * nt;
  int cnt[kClasses] = {};
  for (int64_t t0 = 0; t0 < nt; t0 += 64) {
    const int64_t t = t0 + lane;
    int ci = -1;
    if (t < nt) {
      // 32-bit: the host checks L * B * row tiles < 2^31
      const uint32_t b = ((uint32_t)t / (uint32_t)a.rtiles) % (uint32_t)a.B;
      ci = class_of((a.B <= kColsLds ? ncols_s[b] : a.ncols[b]) + 1);
    }
#pragma unroll
    for (int c = 0; c < kClasses; ++c) {
      const uint64_t m = __ballot(ci == c);
      if (ci == c) {
        const int pos = cnt[c] + __popcll(m & below);
        list[c * nt + pos] = (int)t;
        idx[t] = pos;
      }
      cnt[c] += __popcll(m);
    }
  }
  if (lane < kClasses) {
    int n = 0, slots = 0;
#pragma unroll
    for (int c = 0; c < kClasses; ++c)
      if (c == lane) {
        n = cnt[c];
        slots = a.plan.slots[c];
      }
    // row-tile pairs (class 0): the K-split is chosen for the pair count and
    // stored as the number of 4-split quads (what reaches the partial sums).
    // A workgroup holds 4 pairs, so the pairs count in whole quads: with a
    // partly filled last quad, np pairs would let ceil(np / 4) x KSq
    // workgroups exceed the one-per-CU residency and run a second round.
    const bool pairs = lane == 0 && a.plan.pair0;
    const int64_t units = pairs ? 4 * (((n / a.rtiles) * ((a.rtiles + 1) >> 1) + 3) >> 2) : (int64_t)n;
    int64_t ks = units > 0 ? slots / units : 1;
    ks = ks < 1 ? 1 : (ks > a.plan.ks_max ? a.plan.ks_max : ks);
    if (pairs) ks = ks >= 8 ? ks >> 2 : 1;
    // classes 1 and 2: split each task R times finer than the partials that
    // reach memory and add each R consecutive splits in the workgroup, with
    // R the largest power of two up to the workgroup's wave count for which
    // R * floor(ks / R) keeps at least 95% of the waves busy.  Fewer partials
    // mean fewer partial bytes and a shorter sum in finalize (one image of
    // 13 row tiles otherwise takes ~150 splits per task).
    int red = 1;
    if (lane > 0) {
      for (int r = cost_waves(class_nt(lane), false); r >= 2; r >>= 1) {
        const int64_t kp = ks / r;
        if (kp >= 1 && kp * r * 20 >= ks * 19) {
          red = r;
          ks = kp;
          break;
        }
      }
    }
    a.sched[lane] = n;
    a.sched[kClasses + lane] = (int)ks;
    a.sched[kSchedRed + lane] = red;
    if (a.class_counts) __hip_atomic_store(a.class_counts + lane, n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// s == 1: each thread converts 8 consecutive cells.  grid (nblk, B)
__global__ __launch_bounds__(256) void prep_labels_kernel(PrepArgs a) {
  __shared__ uint32_t pres[kPresWords];
  const int64_t b = blockIdx.y;
  if (a.void_found && blockIdx.x == (unsigned)a.nblk) {  // the void check's own column
    if (b == 0) void_check(a);
    return;
  }
  const int64_t HW = a.H * a.W;
  const bool mark = a.pbits != nullptr;
  const int64_t cell0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  int64_t lab[8];
  if (cell0 < a.HWp) {
    const int64_t* src = a.targets + b * HW + cell0;
    if (HW % 8 == 0 && cell0 + 8 <= HW) {  // 64-byte aligned run of 8 labels
#pragma unroll
      for (int k = 0; k < 8; k += 2) {
        const longlong2 v = *(const longlong2*)(src + k);
        lab[k] = v.x;
        lab[k + 1] = v.y;
      }
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) lab[k] = cell0 + k < HW ? src[k] : -1;
    }
  }
  if (mark) {
    pres_clear(pres);
    __syncthreads();
  }
  if (cell0 < a.HWp) {
    uint32_t wv[4];
    int64_t prev = -1;
    const int64_t lane0 = __shfl(lab[0], 0, 64);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const bool valid = (uint64_t)lab[k] < (uint64_t)a.GT_total;
      const uint32_t v = valid ? (uint32_t)lab[k] : (uint32_t)kNoLabel;
      if (k & 1) wv[k >> 1] |= v << 16;
      else wv[k >> 1] = v;
      if (mark && valid && lab[k] != prev && !(k == 0 && lab[0] == lane0 && (threadIdx.x & 63) != 0))
        pres_mark(pres, lab[k]);
      prev = lab[k];
    }
    // no label output: a presence-only pass (the point-sampling front end
    // takes presence from the full label map and labels at the points)
    if (a.lab16) *(uint4*)(a.lab16 + b * a.HWp + cell0) = make_uint4(wv[0], wv[1], wv[2], wv[3]);
  }
  if (mark) {
    __syncthreads();
    pres_store(a, pres, b);
  }
}

// s > 1: one thread per low-res cell, counts[b][lab][cell] (single writer).
// grid (nblk, B)
__global__ __launch_bounds__(256) void prep_counts_kernel(PrepArgs a) {
  __shared__ uint32_t pres[kPresWords];
  const int64_t b = blockIdx.y;
  if (a.void_found && blockIdx.x == (unsigned)a.nblk) {  // the void check's own column
    if (b == 0) void_check(a);
    return;
  }
  const int64_t HW = a.H * a.W;
  const bool mark = a.pbits != nullptr;
  if (mark) {
    pres_clear(pres);
    __syncthreads();
  }
  const int64_t cell = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (cell < HW) {
    const int64_t i = cell / a.W, j = cell % a.W;
    int64_t prev = -1;
    for (int64_t dy = 0; dy < a.s; ++dy) {
      const int64_t* row = a.targets + (b * a.Ht + i * a.s + dy) * a.Wt + j * a.s;
      for (int64_t dx = 0; dx < a.s; ++dx) {
        const int64_t lab = row[dx];
        if ((uint64_t)lab < (uint64_t)a.GT_total) {
          const int64_t e = (b * a.GT_total + lab) * a.HWp + cell;
          if (a.cw == 1) {
            uint8_t* c = a.counts + e;
            *c = (uint8_t)(*c + 1);
          } else {
            uint16_t* c = (uint16_t*)a.counts + e;
            *c = (uint16_t)(*c + 1);
          }
          if (mark && lab != prev) pres_mark(pres, lab);
        }
        prev = lab;
      }
    }
  }
  if (mark) {
    __syncthreads();
    pres_store(a, pres, b);
  }
}

// Workgroup 0: runs once every presence record of the preparation grid is
// in (and zeroes the assignment's finished-image count).  Workgroups 1 ..
// a.fill.blocks: a slice of the gradient's zero fill.
__global__ __launch_bounds__(1024) void prep_columns_kernel(PrepArgs a) {
  if (a.done && blockIdx.x == 0 && threadIdx.x == 0) *a.done = 0;
  if (blockIdx.x > 0) {
    fill_slice(a.fill, blockIdx.x - 1);
    return;
  }
  columns_and_schedule(a);
}

// Preparation workgroups per image (the presence records' count).
int prep_blocks(const Dims& d) {
  return (int)(d.counts_mode ? ceil_div(d.HW, 256) : ceil_div(d.HWp, 256 * 8));
}

int launch_prep(const PrepArgs& a, const Dims& d, hipStream_t st) {
  ProfScope ps_("prep", st);
  int rc;
  if (a.pbits && (a.GT_total > kPresLabels || a.nblk != prep_blocks(d)))
    return fail(ML_EINVAL, "internal: presence records do not fit the preparation grid");
  if (a.sched && a.plan.ntasks >= ((int64_t)1 << 31)) return fail(ML_EINVAL, "too many row tiles");
  // one more workgroup column for the void check
  const dim3 grid((unsigned)prep_blocks(d) + (a.void_found ? 1u : 0u), (unsigned)d.B);
  if (!d.counts_mode) {
    hipLaunchKernelGGL(prep_labels_kernel, grid, dim3(256), 0, st, a);
  } else {
    rc = launch_fill_i32((int*)a.counts, 0, d.B * d.GT_total * d.HWp * d.cw / 4, st);
    if (rc) return rc;
    hipLaunchKernelGGL(prep_counts_kernel, grid, dim3(256), 0, st, a);
  }
  if ((rc = check_launch("prep"))) return rc;
  if (a.pbits) {
    hipLaunchKernelGGL(prep_columns_kernel, dim3(1u + (unsigned)a.fill.blocks), dim3(1024), 0, st, a);
    if ((rc = check_launch("prep_columns"))) return rc;
  }
  return ML_OK;
}

// Preparation workgroups per image of the presence-only pass over a full
// (Hs, Ws) label map.
int prep_blocks_map(int64_t Hs, int64_t Ws) { return (int)ceil_div(ceil_div(Hs * Ws, kStep) * kStep, 256 * 8); }

// Point-sampling front end: GT presence from the full (Hs, Ws) label map (the
// reference's per-image torch.unique of the whole map,
// functions/sigmoid/pw_sigmoid_ce.py:476-484), the u16 labels of the cost
// contraction from the labels under the points (`coords`, (B, P, 2) with
// P = d.HW), then the column pass and schedule.  `a.pbits` holds
// [B][prep_blocks_map(Hs, Ws)][kPresWords] words and `a.nblk` that count.
int launch_prep_points(const PrepArgs& a, const Dims& d, int64_t Hs, int64_t Ws, const float* coords,
                       hipStream_t st) {
  ProfScope ps_("prep", st);
  if (d.counts_mode || d.H != 1 || !a.pbits || !a.lab16)
    return fail(ML_EINVAL, "internal: point preparation needs a 1 x P grid of labels");
  if (a.GT_total > kPresLabels || a.nblk != prep_blocks_map(Hs, Ws))
    return fail(ML_EINVAL, "internal: presence records do not fit the preparation grid");
  if (a.sched && a.plan.ntasks >= ((int64_t)1 << 31)) return fail(ML_EINVAL, "too many row tiles");
  if (d.B > 65535) return fail(ML_EINVAL, "too many images");
  PrepArgs m = a;
  m.lab16 = nullptr;
  m.H = Hs;
  m.W = Ws;
  m.HWp = ceil_div(Hs * Ws, kStep) * kStep;
  hipLaunchKernelGGL(prep_labels_kernel, dim3((unsigned)a.nblk + (a.void_found ? 1u : 0u), (unsigned)d.B),
                     dim3(256), 0, st, m);
  int rc = check_launch("prep");
  if (rc) return rc;
  rc = launch_point_labels(a.targets, coords, d.B, Hs, Ws, d.HW, a.GT_total, nullptr, a.lab16, d.HWp, st);
  if (rc) return rc;
  hipLaunchKernelGGL(prep_columns_kernel, dim3(1u + (unsigned)a.fill.blocks), dim3(1024), 0, st, a);
  return check_launch("prep_columns");
}

}  // namespace ml
