// Point-sampling front end (Mask2Former-style matching on sampled points).
//
// * point_sample_kernel: bilinear sampling of (N, C, H, W) planes at P points
//   per batch entry, the reference's point_sample (functions/utils.py:12-20):
//   torch.nn.functional.grid_sample with grid = 2 * coords - 1, mode
//   bilinear, zero padding, align_corners as given.  Batch entry n reads the
//   coordinates of entry n % coords_batch, so (L, B, Q, H, W) mask logits
//   sample with one (B, P, 2) point set per image (N = L * B, C = Q), as the
//   reference's pairwise sampling costs do (functions/sigmoid/pw_sigmoid_ce.py:
//   489-495, functions/dice/pw_dice_loss.py:235-239).
// * point_labels_kernel: the label under each point with the reference's
//   floor mapping ix = clamp(long(x * (W_t - 1)), 0, W_t - 1)
//   (pw_sigmoid_ce.py:497-502, pw_dice_loss.py:242-245), as int64 and/or as
//   the u16 compact label row the cost contraction reads (labels outside
//   [0, GT_total) -> no label).
//
// Planes of up to 64 KB are staged in LDS (point_sample_lds_kernel: each
// plane read from HBM once with coalesced loads, the corners gathered from
// LDS); larger planes gather their corners straight from memory
// (point_sample_kernel).  The samples are written along the point index.
#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>

#include "ml_internal.h"

namespace ml {

template <int DT>
__device__ __forceinline__ float ld_val(const void* base, int64_t i) {
  if constexpr (DT == ML_F32) return ((const float*)base)[i];
  else if constexpr (DT == ML_BF16) return bf16_lo((uint32_t)((const uint16_t*)base)[i]);
  else return (float)__builtin_bit_cast(_Float16, ((const uint16_t*)base)[i]);
}

template <int DT>
__device__ __forceinline__ void st_val(void* base, int64_t i, float v) {
  if constexpr (DT == ML_F32) ((float*)base)[i] = v;
  else if constexpr (DT == ML_BF16) ((uint16_t*)base)[i] = (uint16_t)(pack_bf16x2(v, 0.f) & 0xFFFFu);
  else ((uint16_t*)base)[i] = __builtin_bit_cast(uint16_t, (_Float16)v);
}

// Source index of one grid coordinate g in [-1, 1] along a side of `size`
// cells (grid_sample's unnormalisation; written without contraction).
__device__ __forceinline__ float unnormalize(float g, int64_t size, bool align) {
  const float fs = (float)size;
  if (align) return __fmul_rn(__fmul_rn(__fadd_rn(g, 1.f), 0.5f), fs - 1.f);
  return __fmul_rn(__fadd_rn(__fmul_rn(__fadd_rn(g, 1.f), fs), -1.f), 0.5f);
}

constexpr int kPsThreads = 256;
constexpr int kPsChan = 8;  // channels per workgroup (grid z)

// grid (ceil(P / 256), N, ceil(C / kPsChan))
template <int DT>
__global__ __launch_bounds__(kPsThreads) void point_sample_kernel(const void* in, const float* coords,
                                                                   int64_t N, int64_t C, int64_t H,
                                                                   int64_t W, int64_t P, int64_t cb,
                                                                   int align, void* out) {
  const int64_t p = (int64_t)blockIdx.x * kPsThreads + threadIdx.x;
  const int64_t n = blockIdx.y;
  if (p >= P) return;
  const float* cp = coords + ((n % cb) * P + p) * 2;
  const float gx = __fadd_rn(__fmul_rn(2.f, cp[0]), -1.f);
  const float gy = __fadd_rn(__fmul_rn(2.f, cp[1]), -1.f);
  const float ix = unnormalize(gx, W, align != 0);
  const float iy = unnormalize(gy, H, align != 0);
  float x0f = floorf(ix), y0f = floorf(iy);
  // corners outside [0, W) x [0, H) read zero; non-finite or far-away
  // coordinates leave every corner outside (no float -> int overflow)
  const bool xin = x0f >= -1.f && x0f <= (float)(W - 1);
  const bool yin = y0f >= -1.f && y0f <= (float)(H - 1);
  if (!xin) x0f = -2.f;
  if (!yin) y0f = -2.f;
  const int64_t x0 = (int64_t)x0f, y0 = (int64_t)y0f;
  const float x1f = x0f + 1.f, y1f = y0f + 1.f;
  // weights in grid_sample's form: nw = (x_se - ix) * (y_se - iy), ...
  const float w_nw = (x1f - ix) * (y1f - iy);
  const float w_ne = (ix - x0f) * (y1f - iy);
  const float w_sw = (x1f - ix) * (iy - y0f);
  const float w_se = (ix - x0f) * (iy - y0f);
  const bool ok_x0 = xin && x0 >= 0, ok_x1 = xin && x0 + 1 < W;
  const bool ok_y0 = yin && y0 >= 0, ok_y1 = yin && y0 + 1 < H;
  const bool k_nw = ok_x0 && ok_y0, k_ne = ok_x1 && ok_y0;
  const bool k_sw = ok_x0 && ok_y1, k_se = ok_x1 && ok_y1;
  const int64_t o_nw = y0 * W + x0;
  const int64_t HW = H * W;
  const int64_t c0 = (int64_t)blockIdx.z * kPsChan;
  const int64_t c1 = min(C, c0 + kPsChan);
  for (int64_t c = c0; c < c1; ++c) {
    const int64_t base = (n * C + c) * HW + o_nw;
    // the four corner loads of a channel are independent of the previous
    // channel's, so consecutive iterations overlap
    const float v_nw = k_nw ? ld_val<DT>(in, base) : 0.f;
    const float v_ne = k_ne ? ld_val<DT>(in, base + 1) : 0.f;
    const float v_sw = k_sw ? ld_val<DT>(in, base + W) : 0.f;
    const float v_se = k_se ? ld_val<DT>(in, base + W + 1) : 0.f;
    float acc = 0.f;
    if (k_nw) acc += v_nw * w_nw;
    if (k_ne) acc += v_ne * w_ne;
    if (k_sw) acc += v_sw * w_sw;
    if (k_se) acc += v_se * w_se;
    st_val<DT>(out, (n * C + c) * P + p, acc);
  }
}

// LDS-staged form for planes that fit: a workgroup reads CPW planes of one
// batch entry into LDS with coalesced 16-byte loads (each plane from HBM
// once), then gathers every point's four corners from LDS and writes the
// samples along the point index.  The corner weights of a point are formed
// once for its CPW planes.  grid (N * ceil(C / CPW)), dynamic LDS
// CPW * H * W elements.
constexpr int kPsLdsThreads = 1024;
constexpr size_t kPsLdsBytes = 64 * 1024;

template <int DT, int CPW>
__global__ __launch_bounds__(kPsLdsThreads) void point_sample_lds_kernel(
    const void* in, const float* coords, int64_t N, int64_t C, int64_t H, int64_t W, int64_t P,
    int64_t cb, int align, void* out) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  using E = typename std::conditional<DT == ML_F32, float, uint16_t>::type;
  E* plane = (E*)lds_raw;
  const int64_t ngrp = ceil_div(C, (int64_t)CPW);
  const int64_t n = blockIdx.x / ngrp;
  const int64_t c0 = (blockIdx.x % ngrp) * CPW;
  const int ncp = (int)min((int64_t)CPW, C - c0);
  const int64_t HW = H * W;
  // planes c0 .. c0 + ncp - 1 of entry n are contiguous in the input
  const E* src = (const E*)in + (n * C + c0) * HW;
  const int64_t total = (int64_t)ncp * HW;
  constexpr int kPer16 = 16 / sizeof(E);
  if (((uintptr_t)src & 15) == 0) {
    const int64_t n16 = total / kPer16;
    for (int64_t i = threadIdx.x; i < n16; i += kPsLdsThreads) ((uint4*)plane)[i] = ((const uint4*)src)[i];
    for (int64_t i = n16 * kPer16 + threadIdx.x; i < total; i += kPsLdsThreads) plane[i] = src[i];
  } else {
    for (int64_t i = threadIdx.x; i < total; i += kPsLdsThreads) plane[i] = src[i];
  }
  __syncthreads();
  const float* cbase = coords + (n % cb) * P * 2;
  const bool al = align != 0;
  for (int64_t p = threadIdx.x; p < P; p += kPsLdsThreads) {
    const float2 cp = *(const float2*)(cbase + p * 2);
    const float gx = __fadd_rn(__fmul_rn(2.f, cp.x), -1.f);
    const float gy = __fadd_rn(__fmul_rn(2.f, cp.y), -1.f);
    const float ix = unnormalize(gx, W, al);
    const float iy = unnormalize(gy, H, al);
    float x0f = floorf(ix), y0f = floorf(iy);
    const bool xin = x0f >= -1.f && x0f <= (float)(W - 1);
    const bool yin = y0f >= -1.f && y0f <= (float)(H - 1);
    if (!xin) x0f = -2.f;
    if (!yin) y0f = -2.f;
    const int x0 = (int)x0f, y0 = (int)y0f;
    const float x1f = x0f + 1.f, y1f = y0f + 1.f;
    const float w_nw = (x1f - ix) * (y1f - iy);
    const float w_ne = (ix - x0f) * (y1f - iy);
    const float w_sw = (x1f - ix) * (iy - y0f);
    const float w_se = (ix - x0f) * (iy - y0f);
    const bool ok_x0 = xin && x0 >= 0, ok_x1 = xin && x0 + 1 < W;
    const bool ok_y0 = yin && y0 >= 0, ok_y1 = yin && y0 + 1 < H;
    const bool k_nw = ok_x0 && ok_y0, k_ne = ok_x1 && ok_y0;
    const bool k_sw = ok_x0 && ok_y1, k_se = ok_x1 && ok_y1;
    // LDS indices, clamped into the plane for corners outside it (their
    // values are then discarded, not multiplied)
    const int i_nw = k_nw ? y0 * (int)W + x0 : 0;
    const int i_ne = k_ne ? y0 * (int)W + x0 + 1 : 0;
    const int i_sw = k_sw ? (y0 + 1) * (int)W + x0 : 0;
    const int i_se = k_se ? (y0 + 1) * (int)W + x0 + 1 : 0;
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      if (j < ncp) {
        const E* pl = plane + (int64_t)j * HW;
        const float v_nw = ld_val<DT>(pl, i_nw), v_ne = ld_val<DT>(pl, i_ne);
        const float v_sw = ld_val<DT>(pl, i_sw), v_se = ld_val<DT>(pl, i_se);
        float acc = 0.f;
        if (k_nw) acc += v_nw * w_nw;
        if (k_ne) acc += v_ne * w_ne;
        if (k_sw) acc += v_sw * w_sw;
        if (k_se) acc += v_se * w_se;
        st_val<DT>(out, (n * C + c0 + j) * P + p, acc);
      }
    }
  }
}

template <int DT>
static int launch_point_sample_lds(const void* in, const float* coords, int64_t N, int64_t C,
                                   int64_t H, int64_t W, int64_t P, int64_t cb, int align,
                                   void* out, hipStream_t st) {
  const size_t eb = DT == ML_F32 ? 4 : 2;
  const size_t plane = (size_t)H * W * eb;
  const int64_t fit = (int64_t)(kPsLdsBytes / plane);
  const int cpw = (int)std::min<int64_t>({4, fit, C});
  const int64_t blocks = N * ceil_div(C, (int64_t)cpw);
  if (blocks > INT32_MAX) return fail(ML_EINVAL, "point_sample: too many planes");
  const size_t lds = (size_t)cpw * plane;
  const dim3 grid((unsigned)blocks), blk(kPsLdsThreads);
  switch (cpw) {
    case 1: hipLaunchKernelGGL((point_sample_lds_kernel<DT, 1>), grid, blk, lds, st, in, coords, N, C, H, W, P, cb, align, out); break;
    case 2: hipLaunchKernelGGL((point_sample_lds_kernel<DT, 2>), grid, blk, lds, st, in, coords, N, C, H, W, P, cb, align, out); break;
    case 3: hipLaunchKernelGGL((point_sample_lds_kernel<DT, 3>), grid, blk, lds, st, in, coords, N, C, H, W, P, cb, align, out); break;
    default: hipLaunchKernelGGL((point_sample_lds_kernel<DT, 4>), grid, blk, lds, st, in, coords, N, C, H, W, P, cb, align, out); break;
  }
  return check_launch("point_sample");
}

int launch_point_sample(int dtype, const void* in, const float* coords, int64_t N, int64_t C,
                        int64_t H, int64_t W, int64_t P, int64_t cb, int align, void* out,
                        hipStream_t st) {
  if (N == 0 || C == 0 || P == 0) return ML_OK;
  ProfScope ps_("point_sample", st);
  // planes that fit the workgroup's LDS budget are staged there; larger ones
  // gather straight from memory
  const size_t eb = dtype == ML_F32 ? 4 : 2;
  if ((size_t)H * W * eb <= kPsLdsBytes) {
    switch (dtype) {
      case ML_F32: return launch_point_sample_lds<ML_F32>(in, coords, N, C, H, W, P, cb, align, out, st);
      case ML_BF16: return launch_point_sample_lds<ML_BF16>(in, coords, N, C, H, W, P, cb, align, out, st);
      default: return launch_point_sample_lds<ML_F16>(in, coords, N, C, H, W, P, cb, align, out, st);
    }
  }
  const int64_t gz = ceil_div(C, kPsChan);
  if (N > 65535 || gz > 65535) return fail(ML_EINVAL, "point_sample: batch or channel count too large");
  const dim3 grid((unsigned)ceil_div(P, kPsThreads), (unsigned)N, (unsigned)gz);
  switch (dtype) {
    case ML_F32:
      hipLaunchKernelGGL(point_sample_kernel<ML_F32>, grid, dim3(kPsThreads), 0, st, in, coords, N, C,
                         H, W, P, cb, align, out);
      break;
    case ML_BF16:
      hipLaunchKernelGGL(point_sample_kernel<ML_BF16>, grid, dim3(kPsThreads), 0, st, in, coords, N,
                         C, H, W, P, cb, align, out);
      break;
    case ML_F16:
      hipLaunchKernelGGL(point_sample_kernel<ML_F16>, grid, dim3(kPsThreads), 0, st, in, coords, N, C,
                         H, W, P, cb, align, out);
      break;
    default: return fail(ML_EINVAL, "point_sample: unsupported dtype");
  }
  return check_launch("point_sample");
}

// ---- gradient with respect to the sampled planes --------------------------------
// grid_sample's input gradient: every sample's gradient is added to its four
// corner cells with its bilinear weights (corners outside the plane take
// nothing).  Three forms:
// * grouped ((H + 1)(W + 1) <= 16,900, as for 128 x 128 planes, W <= 1151,
//   up to 16,384 points, at least kCsrMinPlanes planes per coordinate set): the
//   points of each coordinate set are sorted into buckets by their base cell
//   once (corner_csr_kernel: a count per bucket in LDS, a scan, a scatter),
//   then each plane's workgroup stages its point gradients in LDS and sums
//   every cell's contributions with no atomics (point_sample_bwd_csr_kernel).
//   The points of one bucket are summed in the order the scatter placed
//   them, which can change between runs, as the order of the reference's
//   CUDA atomics does.
// * LDS float atomics per plane (point_sample_bwd_lds_kernel) for planes of
//   up to 64 KB of accumulators otherwise.
// * global float atomics into a float workspace and a conversion pass for
//   larger planes.
// On 800 planes of 128 x 128 with 12,544 points and 20% of the rows nonzero
// (configuration 2), the grouped form takes 102 us (bucket sort 34 us, gather
// 68 us) against 146 us for the LDS atomics (38 us with plain, racy adds:
// the atomics bind it); global float atomics take 1.9 ms, and a radix sort
// of the corner entries (18 launches) took 110 us alone.  Samples with a
// zero gradient add nothing in the atomic forms; a plane whose gradient row
// is all zero is written as zeros at once in the grouped form.
// I: the index type (int64_t, or int where H * W and its bucket grid fit).
template <typename I = int64_t>
struct Corners {
  I i[4];
  float w[4];
  bool k[4];
  I x0, y0;  // the nw corner, in [-1, W - 1] x [-1, H - 1] when some k[q] holds
};

template <typename I = int64_t>
__device__ __forceinline__ Corners<I> corners_of(const float* cp, I H, I W, bool al) {
  Corners<I> c;
  const float gx = __fadd_rn(__fmul_rn(2.f, cp[0]), -1.f);
  const float gy = __fadd_rn(__fmul_rn(2.f, cp[1]), -1.f);
  const float ix = unnormalize(gx, W, al);
  const float iy = unnormalize(gy, H, al);
  float x0f = floorf(ix), y0f = floorf(iy);
  const bool xin = x0f >= -1.f && x0f <= (float)(W - 1);
  const bool yin = y0f >= -1.f && y0f <= (float)(H - 1);
  if (!xin) x0f = -2.f;
  if (!yin) y0f = -2.f;
  const I x0 = (I)x0f, y0 = (I)y0f;
  const float x1f = x0f + 1.f, y1f = y0f + 1.f;
  c.w[0] = (x1f - ix) * (y1f - iy);  // nw
  c.w[1] = (ix - x0f) * (y1f - iy);  // ne
  c.w[2] = (x1f - ix) * (iy - y0f);  // sw
  c.w[3] = (ix - x0f) * (iy - y0f);  // se
  const bool ok_x0 = xin && x0 >= 0, ok_x1 = xin && x0 + 1 < W;
  const bool ok_y0 = yin && y0 >= 0, ok_y1 = yin && y0 + 1 < H;
  c.k[0] = ok_x0 && ok_y0;
  c.k[1] = ok_x1 && ok_y0;
  c.k[2] = ok_x0 && ok_y1;
  c.k[3] = ok_x1 && ok_y1;
  c.x0 = x0;
  c.y0 = y0;
  c.i[0] = y0 * W + x0;
  c.i[1] = c.i[0] + 1;
  c.i[2] = c.i[0] + W;
  c.i[3] = c.i[2] + 1;
  return c;
}

constexpr int kPsBwdThreads = 512;
constexpr int kPsBwdBatch = 8;
constexpr size_t kPsBwdLdsBytes = 64 * 1024;  // float accumulators of one plane

// One workgroup per plane: accumulate in LDS, then write the plane's
// gradient in the input dtype (every cell, so no clearing is needed).
template <int DT>
__global__ __launch_bounds__(kPsBwdThreads) void point_sample_bwd_lds_kernel(
    const void* gout, const float* coords, int64_t C, int64_t H, int64_t W, int64_t P, int64_t cb,
    int align, void* gin) {
  extern __shared__ __align__(16) float accs[];
  const int64_t plane = blockIdx.x;
  const int64_t n = plane / C;
  const int64_t HW = H * W;
  for (int64_t i = threadIdx.x; i < HW; i += kPsBwdThreads) accs[i] = 0.f;
  __syncthreads();
  const float* cbase = coords + (n % cb) * P * 2;
  const bool al = align != 0;
  // kPsBwdBatch points per thread per round: their gradient and coordinate
  // loads are issued together; samples with a zero gradient add nothing (the
  // rows of unmatched queries are all zero)
  for (int64_t p0 = 0; p0 < P; p0 += (int64_t)kPsBwdThreads * kPsBwdBatch) {
    float g[kPsBwdBatch];
    float2 cp[kPsBwdBatch];
#pragma unroll
    for (int u = 0; u < kPsBwdBatch; ++u) {
      const int64_t p = p0 + (int64_t)u * kPsBwdThreads + threadIdx.x;
      g[u] = p < P ? ld_val<DT>(gout, plane * P + p) : 0.f;
      cp[u] = p < P ? *(const float2*)(cbase + p * 2) : make_float2(0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < kPsBwdBatch; ++u) {
      if (g[u] != 0.f) {
        const float c2[2] = {cp[u].x, cp[u].y};
        const Corners<> c = corners_of(c2, H, W, al);
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (c.k[q]) atomicAdd(&accs[c.i[q]], c.w[q] * g[u]);
      }
    }
  }
  __syncthreads();
  for (int64_t i = threadIdx.x; i < HW; i += kPsBwdThreads) st_val<DT>(gin, plane * HW + i, accs[i]);
}

// Grouped form.  A point whose bilinear footprint touches the plane has a
// base cell (y0, x0) = (floor(iy), floor(ix)) in [-1, H - 1] x [-1, W - 1]:
// bucket (y0 + 1) (W + 1) + (x0 + 1) of NB = (H + 1)(W + 1).  corner_csr_kernel
// sorts each coordinate set's points into their buckets (a count per bucket in
// LDS, a scan, a scatter); record k of set n (buckets in order, bucket b at
// [off[b], off[b + 1])) is point pt[k] with its four corner weights wt[k] =
// (nw, ne, sw, se).  Cell (y, x) is the nw corner of bucket (y, x), the ne
// corner of bucket (y, x - 1), the sw corner of (y - 1, x) and the se corner
// of (y - 1, x - 1): two runs of adjacent buckets, so a cell reads two
// contiguous record ranges.  A corner outside the plane belongs to no cell,
// so its weight is never read.
constexpr int kCsrThreads = 1024;
constexpr int64_t kCsrMaxBuckets = 16900;  // per-bucket counters in LDS (66 KB): 129 x 129 cells
constexpr int64_t kCsrMaxPoints = 16384;   // a plane's point gradients in LDS (64 KB)
constexpr int64_t kCsrMinPlanes = 8;       // planes per coordinate set that repay the grouping
constexpr int kCsrPointsPerThread = (int)(kCsrMaxPoints / kCsrThreads);

constexpr int kBandBuckets = 2304;  // bucket offsets staged per band of the gather at most
static bool csr_form(int64_t C, int64_t H, int64_t W, int64_t P) {
  return (H + 1) * (W + 1) <= kCsrMaxBuckets && 2 * (W + 1) <= kBandBuckets && P <= kCsrMaxPoints &&
         C >= kCsrMinPlanes;
}
struct CsrLayout {
  size_t off, pt, wt, total;  // [cb][NB + 1] u32, [cb][P] u32, [cb][P] float4
};
static CsrLayout csr_layout(int64_t H, int64_t W, int64_t P, int64_t cb) {
  CsrLayout l;
  l.off = 0;
  l.pt = align256((size_t)cb * ((H + 1) * (W + 1) + 1) * 4);
  l.wt = l.pt + align256((size_t)cb * P * 4);
  l.total = l.wt + (size_t)cb * P * 16;
  return l;
}

// One workgroup per coordinate set.
__global__ __launch_bounds__(kCsrThreads) void corner_csr_kernel(const float* coords, int H, int W, int P,
                                                                 int align, uint32_t* off_all,
                                                                 uint32_t* pt_all, float4* wt_all) {
  __shared__ uint32_t cnt[kCsrMaxBuckets];
  __shared__ uint32_t wsum[kCsrThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t set = blockIdx.x;
  const int NB = (H + 1) * (W + 1);
  const float* cs = coords + set * P * 2;
  uint32_t* off = off_all + set * (NB + 1);
  uint32_t* pt = pt_all + set * P;
  float4* wt = wt_all + set * P;
  const bool al = align != 0;
  // the set's points, kCsrPointsPerThread per thread, all loads issued at once
  // (and again for the scatter, from the cache, rather than held across the scan)
  float2 xy[kCsrPointsPerThread];
  auto load_points = [&]() {
#pragma unroll
    for (int u = 0; u < kCsrPointsPerThread; ++u) {
      const int p = u * kCsrThreads + tid;
      xy[u] = p < P ? *(const float2*)(cs + 2 * p) : make_float2(0.f, 0.f);
    }
  };
  load_points();
  for (int i = tid; i < NB; i += kCsrThreads) cnt[i] = 0u;
  __syncthreads();
  int bk[kCsrPointsPerThread];  // the point's bucket, -1 when no corner is in the plane
#pragma unroll
  for (int u = 0; u < kCsrPointsPerThread; ++u) {
    const int p = u * kCsrThreads + tid;
    const float c2[2] = {xy[u].x, xy[u].y};
    const Corners<int> c = corners_of<int>(c2, H, W, al);
    const bool any = c.k[0] | c.k[1] | c.k[2] | c.k[3];
    bk[u] = p < P && any ? (c.y0 + 1) * (W + 1) + (c.x0 + 1) : -1;
    if (bk[u] >= 0) atomicAdd(&cnt[bk[u]], 1u);
  }
  __syncthreads();
  // thread t scans the run of R consecutive buckets starting at t R
  const int R = (NB + kCsrThreads - 1) / kCsrThreads, b0 = tid * R;
  uint32_t run = 0;
  for (int k = 0; k < R; ++k)
    if (b0 + k < NB) run += cnt[b0 + k];
  uint32_t incl = run;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t t = __shfl_up(incl, d, 64);
    if (lane >= d) incl += t;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  uint32_t pos = incl - run, total = 0;
  for (int w = 0; w < kCsrThreads / 64; ++w) {
    pos += w < wave ? wsum[w] : 0u;
    total += wsum[w];
  }
  for (int k = 0; k < R; ++k)
    if (b0 + k < NB) {
      const uint32_t n = cnt[b0 + k];
      off[b0 + k] = pos;
      cnt[b0 + k] = pos;  // the bucket's next free record
      pos += n;
    }
  if (tid == 0) off[NB] = total;
  load_points();
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kCsrPointsPerThread; ++u) {
    if (bk[u] < 0) continue;
    const int p = u * kCsrThreads + tid;
    const float c2[2] = {xy[u].x, xy[u].y};
    const Corners<int> c = corners_of<int>(c2, H, W, al);
    const uint32_t at = atomicAdd(&cnt[bk[u]], 1u);
    pt[at] = (uint32_t)p;
    wt[at] = make_float4(c.w[0], c.w[1], c.w[2], c.w[3]);
  }
}

// One workgroup per plane: its point gradients into LDS (a gradient row that
// is all zero writes a zero plane at once), then bands of RB cell rows.  The
// buckets a band reads (rows y0 - 1 .. y0 + RB - 1) are consecutive, and so
// are their records: the band's offsets and records are staged in LDS, and
// each thread sums its cells' two record ranges there (a band with more than
// kBandRecords records reads them from memory).  The next band's offsets
// and records are loaded into registers while the current band is summed.
// Every cell of the plane is written.  Indices are 32-bit: at most 16,900
// buckets, 16,384 points and as many records per coordinate set.
constexpr int kBandRecords = 3072;  // 60 KB of staged records
constexpr int kBandCells = 2048;    // cells per band (at least one row)
constexpr int kBandU = kBandRecords / kCsrThreads;             // records per thread
constexpr int kBandOffU = (kBandBuckets + kCsrThreads) / kCsrThreads;  // offsets per thread
template <int DT>
__global__ __launch_bounds__(kCsrThreads) void point_sample_bwd_csr_kernel(
    const void* gout, int C, int H, int W, int P, int cb, int RB, const uint32_t* off_all,
    const uint32_t* pt_all, const float4* wt_all, void* gin) {
  extern __shared__ __align__(16) unsigned char sm[];
  float4* rw = (float4*)sm;                       // [kBandRecords] weights
  uint32_t* rp = (uint32_t*)(rw + kBandRecords);  // [kBandRecords] points
  uint32_t* bo = rp + kBandRecords;               // [kBandBuckets + 1] offsets
  float* g = (float*)(bo + kBandBuckets + 4);     // [P]
  const int tid = threadIdx.x;
  const int W1 = W + 1, HW = H * W;
  const int64_t plane = blockIdx.x, obase = plane * HW;
  const int set = (int)((plane / C) % cb);
  int nz = 0;
  {
    float v[kCsrPointsPerThread];  // all loads issued at once
#pragma unroll
    for (int u = 0; u < kCsrPointsPerThread; ++u) {
      const int p = u * kCsrThreads + tid;
      v[u] = p < P ? ld_val<DT>(gout, plane * P + p) : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kCsrPointsPerThread; ++u) {
      const int p = u * kCsrThreads + tid;
      if (p < P) g[p] = v[u];
      nz |= v[u] != 0.f;
    }
  }
  if (!__syncthreads_or(nz)) {
    for (int i = tid; i < HW; i += kCsrThreads) st_val<DT>(gin, obase + i, 0.f);
    return;
  }
  const uint32_t* off = off_all + (int64_t)set * ((H + 1) * W1 + 1);
  const uint32_t* pt = pt_all + (int64_t)set * P;
  const float4* wt = wt_all + (int64_t)set * P;
  // band y0 reads buckets [y0 W1, (y0 + rows + 1) W1): nbk + 1 offsets from y0 W1
  auto nbk_of = [&](int y0) { return (min(RB, H - y0) + 1) * W1; };
  // Registers that carry the next band (kBandOffU = kBandU = 3 per thread,
  // named rather than arrays, so that they stay in registers across the sum):
  // its offsets and records, loaded with unconditional loads at clamped
  // indices (the set's arrays hold (H + 1) W1 + 1 offsets and P records).
  static_assert(kBandOffU == 3 && kBandU == 3, "three carried slots per thread");
  uint32_t no0, no1, no2, nq0, nq1, nq2;
  float4 nw0, nw1, nw2;
  const uint32_t last = (uint32_t)P - 1u;
  auto fetch = [&](int y0) {
    const int nbk = nbk_of(y0);
    const uint32_t* o = off + y0 * W1;
    const uint32_t r0 = o[0];  // wave-uniform
    no0 = o[min(tid, nbk)];
    no1 = o[min(kCsrThreads + tid, nbk)];
    no2 = o[min(2 * kCsrThreads + tid, nbk)];
    const uint32_t k0 = min(r0 + (uint32_t)tid, last), k1 = min(r0 + (uint32_t)(kCsrThreads + tid), last),
                   k2 = min(r0 + (uint32_t)(2 * kCsrThreads + tid), last);
    nq0 = pt[k0];
    nq1 = pt[k1];
    nq2 = pt[k2];
    nw0 = wt[k0];
    nw1 = wt[k1];
    nw2 = wt[k2];
  };
  // every slot of the staging room is written (past the band's records and
  // offsets with entries that no cell reads)
  auto stage = [&]() {
    bo[tid] = no0;
    bo[kCsrThreads + tid] = no1;
    if (2 * kCsrThreads + tid <= kBandBuckets) bo[2 * kCsrThreads + tid] = no2;
    rp[tid] = nq0;
    rp[kCsrThreads + tid] = nq1;
    rp[2 * kCsrThreads + tid] = nq2;
    rw[tid] = nw0;
    rw[kCsrThreads + tid] = nw1;
    rw[2 * kCsrThreads + tid] = nw2;
  };
  fetch(0);
  stage();
  __syncthreads();
  for (int y0 = 0; y0 < H; y0 += RB) {
    const int rows = min(RB, H - y0), nbk = nbk_of(y0);
    const uint32_t r0 = bo[0], nr = bo[nbk] - r0;
    const bool staged = nr <= (uint32_t)kBandRecords;
    if (y0 + RB < H) fetch(y0 + RB);  // lands while this band is summed
    const int ncell = rows * W;
    for (int k = tid; k < ncell; k += kCsrThreads) {
      const int yl = k / W, x = k - yl * W;
      // local bucket (y, x) of the band: (yl + 1) W1 + (x + 1)
      const int bn = (yl + 1) * W1 + (x + 1), bs = bn - W1;
      float acc = 0.f;
      if (staged) {
        // buckets (y, x - 1), (y, x): this cell is their ne and nw corner
        for (uint32_t j = bo[bn - 1] - r0, m = bo[bn] - r0, e = bo[bn + 1] - r0; j < e; ++j)
          acc += (j < m ? rw[j].y : rw[j].x) * g[rp[j]];
        // buckets (y - 1, x - 1), (y - 1, x): its se and sw corner
        for (uint32_t j = bo[bs - 1] - r0, m = bo[bs] - r0, e = bo[bs + 1] - r0; j < e; ++j)
          acc += (j < m ? rw[j].w : rw[j].z) * g[rp[j]];
      } else {
        for (uint32_t j = bo[bn - 1], m = bo[bn], e = bo[bn + 1]; j < e; ++j)
          acc += (j < m ? wt[j].y : wt[j].x) * g[pt[j]];
        for (uint32_t j = bo[bs - 1], m = bo[bs], e = bo[bs + 1]; j < e; ++j)
          acc += (j < m ? wt[j].w : wt[j].z) * g[pt[j]];
      }
      st_val<DT>(gin, obase + (int64_t)y0 * W + k, acc);
    }
    if (y0 + RB < H) {
      __syncthreads();  // every thread is done with this band's LDS
      stage();
      __syncthreads();
    }
  }
}
// Rows per band: at most kBandCells cells and kBandBuckets offsets, and the
// expected records (P / NB per bucket) within half the staging room.
static int csr_band_rows(int64_t H, int64_t W, int64_t P) {
  const double per_bucket = (double)P / (double)((H + 1) * (W + 1));
  int64_t rb = std::min<int64_t>(kBandCells / W, kBandBuckets / (W + 1) - 1);
  const int64_t by_records = (int64_t)(0.5 * kBandRecords / (per_bucket * (W + 1) + 1e-9)) - 1;
  rb = std::min(rb, by_records);
  return (int)std::max<int64_t>(1, std::min<int64_t>(rb, H));
}
static size_t csr_gather_lds(int64_t P) {
  return (size_t)kBandRecords * 20 + (size_t)(kBandBuckets + 4) * 4 + (size_t)P * 4;
}
// The gather's dynamic LDS limit raised to its largest size, once per device
// (the attribute is set with that device current); the lock makes the first
// call of several host threads safe.
template <int DT>
static int csr_raise_lds() {
  constexpr int kMaxDev = 64;
  static std::atomic<int> done[kMaxDev];
  static std::mutex mu;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev)
    return fail(ML_ELAUNCH, "point_sample backward: no current device (or more than 64)");
  if (!done[dev].load(std::memory_order_acquire)) {
    std::lock_guard<std::mutex> g(mu);
    if (!done[dev].load(std::memory_order_relaxed)) {
      const size_t most = csr_gather_lds(kCsrMaxPoints);
      if (hipFuncSetAttribute((const void*)point_sample_bwd_csr_kernel<DT>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)most) != hipSuccess)
        return fail(ML_ELAUNCH, "point_sample backward: cannot raise the LDS limit");
      done[dev].store(1, std::memory_order_release);
    }
  }
  return ML_OK;
}

// Planes too large for LDS: float atomics into a zeroed float buffer, then a
// conversion pass.  grid (ceil(P / 256), N, ceil(C / kPsChan))
template <int DT>
__global__ __launch_bounds__(kPsThreads) void point_sample_bwd_global_kernel(
    const void* gout, const float* coords, int64_t N, int64_t C, int64_t H, int64_t W, int64_t P,
    int64_t cb, int align, float* acc) {
  const int64_t p = (int64_t)blockIdx.x * kPsThreads + threadIdx.x;
  const int64_t n = blockIdx.y;
  if (p >= P) return;
  const Corners<> c = corners_of(coords + ((n % cb) * P + p) * 2, H, W, align != 0);
  const int64_t c0 = (int64_t)blockIdx.z * kPsChan;
  const int64_t c1 = min(C, c0 + kPsChan);
  for (int64_t ch = c0; ch < c1; ++ch) {
    const float g = ld_val<DT>(gout, (n * C + ch) * P + p);
    if (g == 0.f) continue;  // rows of unmatched queries are all zero
    float* a = acc + (n * C + ch) * H * W;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (c.k[q]) unsafeAtomicAdd(&a[c.i[q]], c.w[q] * g);
  }
}

template <int DT>
__global__ __launch_bounds__(256) void f32_to_dtype_kernel(const float* src, void* dst, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    st_val<DT>(dst, i, src[i]);
}

size_t point_sample_bwd_workspace(int dtype, int64_t N, int64_t C, int64_t H, int64_t W, int64_t P,
                                  int64_t cb) {
  (void)dtype;
  if (csr_form(C, H, W, P)) return csr_layout(H, W, P, cb).total;
  if ((size_t)H * W * 4 <= kPsBwdLdsBytes) return 0;
  return (size_t)N * C * H * W * 4;
}

template <int DT>
static int launch_bwd_dt(const void* gout, const float* coords, int64_t N, int64_t C, int64_t H,
                         int64_t W, int64_t P, int64_t cb, int align, void* gin, float* acc,
                         hipStream_t st) {
  const int64_t planes = N * C;
  if (csr_form(C, H, W, P)) {
    if (!acc) return fail(ML_EWORKSPACE, "point_sample backward: a workspace is required");
    if (planes > INT32_MAX || cb > INT32_MAX) return fail(ML_EINVAL, "point_sample backward: too many planes");
    const CsrLayout l = csr_layout(H, W, P, cb);
    unsigned char* w = (unsigned char*)acc;
    uint32_t* off = (uint32_t*)(w + l.off);
    uint32_t* pt = (uint32_t*)(w + l.pt);
    float4* wt = (float4*)(w + l.wt);
    const int64_t sets = std::min(cb, N);  // coordinate sets that some plane reads
    hipLaunchKernelGGL(corner_csr_kernel, dim3((unsigned)sets), dim3(kCsrThreads), 0, st, coords, (int)H,
                       (int)W, (int)P, align, off, pt, wt);
    int rc = check_launch("point_sample_backward");
    if (rc) return rc;
    if ((rc = csr_raise_lds<DT>())) return rc;
    hipLaunchKernelGGL(point_sample_bwd_csr_kernel<DT>, dim3((unsigned)planes), dim3(kCsrThreads),
                       csr_gather_lds(P), st, gout, (int)C, (int)H, (int)W, (int)P, (int)cb,
                       csr_band_rows(H, W, P), (const uint32_t*)off, (const uint32_t*)pt,
                       (const float4*)wt, gin);
    return check_launch("point_sample_backward");
  }
  if ((size_t)H * W * 4 <= kPsBwdLdsBytes) {
    if (planes > INT32_MAX) return fail(ML_EINVAL, "point_sample backward: too many planes");
    hipLaunchKernelGGL(point_sample_bwd_lds_kernel<DT>, dim3((unsigned)planes), dim3(kPsBwdThreads),
                       (size_t)H * W * 4, st, gout, coords, C, H, W, P, cb, align, gin);
    return check_launch("point_sample_backward");
  }
  if (!acc) return fail(ML_EWORKSPACE, "point_sample backward: a float workspace is required");
  const int64_t total = planes * H * W;
  int rc = launch_zero_fill(acc, (size_t)total * 4, st);
  if (rc) return rc;
  const int64_t gz = ceil_div(C, kPsChan);
  if (N > 65535 || gz > 65535) return fail(ML_EINVAL, "point_sample: batch or channel count too large");
  if (P > 0) {
    hipLaunchKernelGGL(point_sample_bwd_global_kernel<DT>,
                       dim3((unsigned)ceil_div(P, kPsThreads), (unsigned)N, (unsigned)gz),
                       dim3(kPsThreads), 0, st, gout, coords, N, C, H, W, P, cb, align, acc);
    if ((rc = check_launch("point_sample_backward"))) return rc;
  }
  const int64_t blocks = std::min<int64_t>(ceil_div(total, 256), 8192);
  hipLaunchKernelGGL(f32_to_dtype_kernel<DT>, dim3((unsigned)std::max<int64_t>(blocks, 1)), dim3(256), 0,
                     st, acc, gin, total);
  return check_launch("point_sample_backward");
}

int launch_point_sample_backward(int dtype, const void* gout, const float* coords, int64_t N,
                                 int64_t C, int64_t H, int64_t W, int64_t P, int64_t cb, int align,
                                 void* gin, float* acc, hipStream_t st) {
  if (N == 0 || C == 0) return ML_OK;
  ProfScope ps_("point_sample_backward", st);
  switch (dtype) {
    case ML_F32: return launch_bwd_dt<ML_F32>(gout, coords, N, C, H, W, P, cb, align, gin, acc, st);
    case ML_BF16: return launch_bwd_dt<ML_BF16>(gout, coords, N, C, H, W, P, cb, align, gin, acc, st);
    case ML_F16: return launch_bwd_dt<ML_F16>(gout, coords, N, C, H, W, P, cb, align, gin, acc, st);
  }
  return fail(ML_EINVAL, "point_sample backward: unsupported dtype");
}

// Index of the cell under coordinate x in [0, 1] along a side of `size`
// cells: long(x * (size - 1)) in float32, truncated toward zero, clamped to
// [0, size - 1]; NaN maps to 0.
__device__ __forceinline__ int64_t point_cell(float x, int64_t size) {
  const float f = __fmul_rn(x, (float)(size - 1));
  if (!(f > 0.f)) return 0;  // also NaN
  if (f >= (float)(size - 1)) return size - 1;
  return (int64_t)f;
}

// grid (ceil(HWp / 256), B): point p < P writes its label; the padding points
// [P, HWp) of the u16 row get no label.
__global__ __launch_bounds__(256) void point_labels_kernel(const int64_t* targets, const float* coords,
                                                           int64_t Ht, int64_t Wt, int64_t P,
                                                           int64_t GT_total, int64_t* out64,
                                                           uint16_t* out16, int64_t HWp) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (p < P) {
    const float* cp = coords + (b * P + p) * 2;
    const int64_t ix = point_cell(cp[0], Wt), iy = point_cell(cp[1], Ht);
    const int64_t lab = targets[(b * Ht + iy) * Wt + ix];
    if (out64) out64[b * P + p] = lab;
    if (out16)
      out16[b * HWp + p] = (uint64_t)lab < (uint64_t)GT_total ? (uint16_t)lab : (uint16_t)kNoLabel;
  } else if (out16 && p < HWp) {
    out16[b * HWp + p] = (uint16_t)kNoLabel;
  }
}

int launch_point_labels(const int64_t* targets, const float* coords, int64_t B, int64_t Ht,
                        int64_t Wt, int64_t P, int64_t GT_total, int64_t* out64, uint16_t* out16,
                        int64_t HWp, hipStream_t st) {
  const int64_t n = out16 ? HWp : P;
  if (B == 0 || n == 0) return ML_OK;
  if (B > 65535) return fail(ML_EINVAL, "point labels: too many images");
  hipLaunchKernelGGL(point_labels_kernel, dim3((unsigned)ceil_div(n, 256), (unsigned)B), dim3(256), 0,
                     st, targets, coords, Ht, Wt, P, GT_total, out64, out16, HWp);
  return check_launch("point_labels");
}

}  // namespace ml
