// Target preparation: int64 label map -> compact per-image target operands.
//
//   s == 1 : u16 label per cell (labels outside [0, GT_total) -> 0xFFFF)
//   s  > 1 : u8 count of each label inside the s x s block of every cell
//            (B, GT_total, HWp), the reference's count tensor
//            (src/cuda/utils.cuh:6-36)
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

// Zero `n16` 16-byte words, then `ntail` trailing bytes.  Streaming
// (non-temporal) stores: the buffer is a gradient that is not read again
// before the backward, so it should not displace the forward's working set
// from the L2.
__global__ __launch_bounds__(256) void zero_fill_kernel(u32x4_t* p, int64_t n16,
                                                        unsigned char* tail, int64_t ntail) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const u32x4_t z = {0u, 0u, 0u, 0u};
  for (; i + 3 * stride < n16; i += 4 * stride) {
    __builtin_nontemporal_store(z, p + i);
    __builtin_nontemporal_store(z, p + i + stride);
    __builtin_nontemporal_store(z, p + i + 2 * stride);
    __builtin_nontemporal_store(z, p + i + 3 * stride);
  }
  for (; i < n16; i += stride) __builtin_nontemporal_store(z, p + i);
  if (blockIdx.x == 0 && threadIdx.x < ntail) tail[threadIdx.x] = 0;
}

// 64 workgroups of 4 waves.  Measured on MI355X beside the assignment kernel
// (375 MB): 64 workgroups still write at the full rate (72 us; 32 take 104 us)
// while touching only a quarter of the CUs, so the latency-bound assignment
// is slowed least (85 us vs. 77 us alone; 119 us beside 1024 workgroups).
constexpr int64_t kFillBlocks = 64;

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

constexpr int kMarkMax = 8192;  // GT slots marked in LDS; more -> direct global marks

// Mark label `lab` present: an LDS byte, or the global flag when the GT count
// exceeds the LDS table.  Lanes of a wave that agree with lane 0 skip the
// store (most cells of a wave carry one label).
__device__ __forceinline__ void mark_present(unsigned char* pres, int* present, int64_t lab,
                                             bool lds) {
  if (lds) pres[lab] = 1;
  else present[lab] = 1;
}

// Compacted list of the columns whose GT is non-empty, one wave per image
// (images w, w + nwaves, ...), then, on wave 0, the cost schedule (per
// column-tile class: its tasks in ascending order, their count and K-split;
// per task: its position in its class list).  Run by one workgroup after the
// target-preparation grid.
__device__ void columns_and_schedule(const PrepArgs& a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nw = blockDim.x >> 6;
  const uint64_t below = (1ull << lane) - 1ull;
  for (int64_t b = wave; b < a.B; b += nw) {
    int base = 0;
    for (int64_t c0 = 0; c0 < a.GT_out; c0 += 64) {
      const int64_t c = c0 + lane;
      bool ok = false;
      if (c < a.GT_out) {
        const int64_t act = c + (c >= a.bg ? 1 : 0);
        ok = a.present[b * a.GT_total + act] != 0;
      }
      const uint64_t m = __ballot(ok);
      const int slot = base + __popcll(m & below);
      if (c < a.GT_out) {
        a.slot_of_col[b * a.GT_out + c] = ok ? slot : -1;
        if (ok) a.colmap[b * a.nslot + slot] = (int)c;
      }
      base += __popcll(m);
    }
    for (int s = base + lane; s < a.nslot; s += 64) a.colmap[b * a.nslot + s] = -1;
    if (lane == 0) a.ncols[b] = base;
  }
  if (!a.sched) return;
  __syncthreads();
  if (wave != 0) return;
  const int64_t nt = a.plan.ntasks;
  int* list = a.sched + 2 * kClasses;
  int* idx = list + kClasses * nt;
  int cnt[kClasses] = {0, 0, 0, 0};
  for (int64_t t0 = 0; t0 < nt; t0 += 64) {
    const int64_t t = t0 + lane;
    int ci = -1;
    if (t < nt) ci = class_of(a.ncols[(t / a.rtiles) % a.B] + 1);
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
    int64_t ks = n > 0 ? slots / n : 1;
    ks = ks < 1 ? 1 : (ks > a.plan.ks_max ? a.plan.ks_max : ks);
    a.sched[lane] = n;
    a.sched[kClasses + lane] = (int)ks;
  }
}

// s == 1: each thread converts 8 consecutive cells.  grid (ceil(HWp/2048), B)
__global__ __launch_bounds__(256) void prep_labels_kernel(PrepArgs a) {
  __shared__ unsigned char pres[kMarkMax];
  const int64_t b = blockIdx.y;
  const int64_t HW = a.H * a.W;
  const bool mark = a.present != nullptr;
  const bool lds = a.GT_total <= kMarkMax;
  int* present = mark ? a.present + b * a.GT_total : nullptr;
  if (mark && lds) {
    for (int i = threadIdx.x; i < a.GT_total; i += blockDim.x) pres[i] = 0;
    __syncthreads();
  }
  const int64_t cell0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (cell0 < a.HWp) {
    int64_t lab[8];
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
        mark_present(pres, present, lab[k], lds);
      prev = lab[k];
    }
    *(uint4*)(a.lab16 + b * a.HWp + cell0) = make_uint4(wv[0], wv[1], wv[2], wv[3]);
  }
  if (mark && lds) {
    __syncthreads();
    for (int i = threadIdx.x; i < a.GT_total; i += blockDim.x)
      if (pres[i]) present[i] = 1;
  }
}

// s > 1: one thread per low-res cell, counts[b][lab][cell] (single writer).
__global__ __launch_bounds__(256) void prep_counts_kernel(PrepArgs a) {
  __shared__ unsigned char pres[kMarkMax];
  const int64_t b = blockIdx.y;
  const int64_t HW = a.H * a.W;
  const bool mark = a.present != nullptr;
  const bool lds = a.GT_total <= kMarkMax;
  int* present = mark ? a.present + b * a.GT_total : nullptr;
  if (mark && lds) {
    for (int i = threadIdx.x; i < a.GT_total; i += blockDim.x) pres[i] = 0;
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
          uint8_t* c = a.counts8 + (b * a.GT_total + lab) * a.HWp + cell;
          *c = (uint8_t)(*c + 1);
          if (mark && lab != prev) mark_present(pres, present, lab, lds);
        }
        prev = lab;
      }
    }
  }
  if (mark && lds) {
    __syncthreads();
    for (int i = threadIdx.x; i < a.GT_total; i += blockDim.x)
      if (pres[i]) present[i] = 1;
  }
}

// One workgroup: runs once every presence mark of the preparation grid is in.
__global__ __launch_bounds__(1024) void prep_columns_kernel(PrepArgs a) { columns_and_schedule(a); }

int launch_prep(const PrepArgs& a, const Dims& d, hipStream_t st) {
  ProfScope ps_("prep", st);
  int rc;
  // presence flags, error word and grid tickets in one fill
  if (a.present && (rc = launch_fill_i32(a.present, 0, a.fill_ints, st))) return rc;
  if (!d.counts_mode) {
    const dim3 grid((unsigned)ceil_div(d.HWp, 256 * 8), (unsigned)d.B);
    hipLaunchKernelGGL(prep_labels_kernel, grid, dim3(256), 0, st, a);
  } else {
    rc = launch_fill_i32((int*)a.counts8, 0, d.B * d.GT_total * d.HWp / 4, st);
    if (rc) return rc;
    const dim3 grid((unsigned)ceil_div(d.HW, 256), (unsigned)d.B);
    hipLaunchKernelGGL(prep_counts_kernel, grid, dim3(256), 0, st, a);
  }
  if ((rc = check_launch("prep"))) return rc;
  if (a.present) {
    hipLaunchKernelGGL(prep_columns_kernel, dim3(1), dim3(1024), 0, st, a);
    if ((rc = check_launch("prep_columns"))) return rc;
  }
  return ML_OK;
}

}  // namespace ml
