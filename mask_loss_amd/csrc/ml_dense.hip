// Non-pairwise (per-class) losses over dense class logits (L, B, C, H, W)
// against an integer label map (B, Ht, Wt), counted per low-resolution cell:
//
//   sigmoid CE (src/cuda/sigmoid_ce.cu:13-332):
//     loss[l] = scale / (num_masks Ht Wt) * sum_{b,c,cell} ap mp cp n + an mn cn (N2 - n)
//     grad    = g[l] scale / (num_masks Ht Wt) *
//               ( -ap n mp (gamma p cp + 1-p) + an (N2-n) mn (gamma (1-p) cn + p) )
//   dice (src/cuda/dice_loss.cu:13-289):
//     I = sum p n, P = sum N2 p, T = sum n   per (l, b, c)
//     loss[l] = scale / num_masks * sum_{b,c} 1 - (2I + smooth) / (P + T + smooth)
//     grad    = -g[l] scale / num_masks * (2 n D - N2 (2I + smooth)) / D^2 * p (1-p),
//               D = P + T + smooth
//
// with n = count of class c inside the s x s target block of the cell.  The
// reference gives every low-resolution cell its own block of 64 threads and
// reads the C logits of that cell with stride H*W; here a workgroup streams a
// contiguous chunk of one (l, b, c) plane (coalesced 16-byte loads) against
// the compact targets (u16 labels for s == 1, u8 / u16 counts for s > 1) shared by
// all planes of the image.  Sums are float64 per workgroup, combined in a
// fixed order by one small kernel, so results are deterministic (the
// reference's float / double atomics are not).
#include "ml_internal.h"

namespace ml {

constexpr int kDenseU = 4;                                 // 8-cell groups per thread
constexpr int64_t kDenseChunk = 256 * 8 * kDenseU;         // cells per workgroup

__device__ __forceinline__ void dense_load8(const void* base, int dt, int64_t i, int64_t nvalid,
                                            bool vec, float z[8]) {
  if (dt == ML_F32) {
    const float* p = (const float*)base + i;
    if (vec && nvalid >= 8) {
      const float4 v0 = *(const float4*)p;
      const float4 v1 = *(const float4*)(p + 4);
      z[0] = v0.x; z[1] = v0.y; z[2] = v0.z; z[3] = v0.w;
      z[4] = v1.x; z[5] = v1.y; z[6] = v1.z; z[7] = v1.w;
    } else {
      for (int k = 0; k < 8; ++k) z[k] = k < nvalid ? p[k] : 0.f;
    }
    return;
  }
  const uint16_t* p = (const uint16_t*)base + i;
  uint32_t w[4];
  if (vec && nvalid >= 8) {
    const uint4 v = *(const uint4*)p;
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else {
    for (int k = 0; k < 4; ++k) {
      const uint32_t lo = 2 * k < nvalid ? p[2 * k] : 0u;
      const uint32_t hi = 2 * k + 1 < nvalid ? p[2 * k + 1] : 0u;
      w[k] = lo | (hi << 16);
    }
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if (dt == ML_BF16) {
      z[2 * k] = bf16_lo(w[k]);
      z[2 * k + 1] = bf16_hi(w[k]);
    } else {
      z[2 * k] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[k] & 0xFFFF));
      z[2 * k + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[k] >> 16));
    }
  }
}

__device__ __forceinline__ void dense_store8(void* base, int dt, int64_t i, const float g[8],
                                             int64_t nvalid, bool vec) {
  if (dt == ML_F32) {
    float* p = (float*)base + i;
    if (vec && nvalid >= 8) {
      *(float4*)p = make_float4(g[0], g[1], g[2], g[3]);
      *(float4*)(p + 4) = make_float4(g[4], g[5], g[6], g[7]);
    } else {
      for (int k = 0; k < 8; ++k)
        if (k < nvalid) p[k] = g[k];
    }
    return;
  }
  uint16_t* p = (uint16_t*)base + i;
  uint32_t w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if (dt == ML_BF16) {
      w[k] = pack_bf16x2(g[2 * k], g[2 * k + 1]);
    } else {
      const uint16_t lo = __builtin_bit_cast(uint16_t, (_Float16)g[2 * k]);
      const uint16_t hi = __builtin_bit_cast(uint16_t, (_Float16)g[2 * k + 1]);
      w[k] = (uint32_t)lo | ((uint32_t)hi << 16);
    }
  }
  if (vec && nvalid >= 8) {
    *(uint4*)p = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
    for (int k = 0; k < 8; ++k)
      if (k < nvalid) p[k] = (uint16_t)(w[k >> 1] >> ((k & 1) * 16));
  }
}

// counts of class c for 8 cells starting at cell0
__device__ __forceinline__ void dense_count8(const DenseArgs& a, int64_t b, int64_t c,
                                             int64_t cell0, float n[8]) {
  if (a.counts == nullptr) {
    const uint4 lv = *(const uint4*)(a.lab16 + b * a.HWp + cell0);
    const uint32_t w[4] = {lv.x, lv.y, lv.z, lv.w};
    const uint32_t c32 = (uint32_t)c;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      n[2 * k] = (w[k] & 0xFFFFu) == c32 ? 1.f : 0.f;
      n[2 * k + 1] = (w[k] >> 16) == c32 ? 1.f : 0.f;
    }
  } else {
    counts8_f(a.counts, a.cw, (b * a.C + c) * a.HWp + cell0, n);
  }
}

__device__ __forceinline__ double block_sum_d(double v, double* sh) {
  v = wave_sum_d(v);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) sh[wave] = v;
  __syncthreads();
  return (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

// Forward partial sums of one chunk of one (l, b, c) plane.
// grid (nchunk, C, L*B); partials[(lb*C + c)*nchunk + chunk][np]
template <bool DICE>
__global__ __launch_bounds__(256) void dense_fwd_kernel(DenseArgs a, int64_t nchunk) {
  __shared__ double sh[3][4];
  const int64_t chunk = blockIdx.x, c = blockIdx.y, lb = blockIdx.z;
  const int64_t b = lb % a.B;
  const int64_t plane = (lb * a.C + c) * a.HW;
  const bool vec = a.dtype == ML_F32 ? (a.HW % 4 == 0) : (a.HW % 8 == 0);
  double s0 = 0.0, s1 = 0.0, s2 = 0.0;
  const int64_t c0 = chunk * kDenseChunk + (int64_t)threadIdx.x * 8;
  float z[kDenseU][8], n[kDenseU][8];
#pragma unroll
  for (int u = 0; u < kDenseU; ++u) {
    const int64_t cell0 = c0 + u * 256 * 8;
    if (cell0 < a.HW) {
      dense_load8(a.logits, a.dtype, plane + cell0, a.HW - cell0, vec, z[u]);
      dense_count8(a, b, c, cell0, n[u]);
    }
  }
#pragma unroll
  for (int u = 0; u < kDenseU; ++u) {
    const int64_t cell0 = c0 + u * 256 * 8;
    if (cell0 >= a.HW) continue;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (cell0 + k >= a.HW) continue;
      const Sig sg = sig_terms(z[u][k]);
      const float nk = n[u][k];
      if constexpr (DICE) {
        s0 += (double)(sg.p * nk);     // I
        s1 += (double)(a.N2 * sg.p);   // P
        s2 += (double)nk;              // T
      } else {
        float mn, mp;
        focal_mods(sg, a.ep, mn, mp);
        const float lp = a.ep.ap * mp * sg.cp * nk;
        const float ln = a.ep.an * mn * sg.cn * (a.N2 - nk);
        s0 += (double)(lp + ln);
      }
    }
  }
  double* out = a.partials + ((lb * a.C + c) * nchunk + chunk) * (DICE ? 3 : 1);
  s0 = block_sum_d(s0, sh[0]);
  if constexpr (DICE) {
    s1 = block_sum_d(s1, sh[1]);
    s2 = block_sum_d(s2, sh[2]);
  }
  if (threadIdx.x == 0) {
    out[0] = s0;
    if constexpr (DICE) {
      out[1] = s1;
      out[2] = s2;
    }
  }
}

// Fixed-order reduction, one workgroup per layer.
//   sigmoid: loss[l] = scale * sum / (num_masks Ht Wt)
//   dice: I, P, T per (l, b, c) (float), loss[l] = scale / num_masks * sum (1 - dice)
template <bool DICE>
__global__ __launch_bounds__(256) void dense_reduce_kernel(DenseArgs a, int64_t nchunk) {
  __shared__ double sh[4];
  const int64_t l = blockIdx.x;
  const int64_t planes = a.B * a.C;
  double acc = 0.0;
  for (int64_t pl = threadIdx.x; pl < planes; pl += 256) {
    const double* src = a.partials + ((l * planes + pl) * nchunk) * (DICE ? 3 : 1);
    if constexpr (DICE) {
      double I = 0.0, P = 0.0, T = 0.0;
      for (int64_t k = 0; k < nchunk; ++k) {
        I += src[3 * k];
        P += src[3 * k + 1];
        T += src[3 * k + 2];
      }
      const int64_t o = l * planes + pl;
      a.I_out[o] = (float)I;
      a.P_out[o] = (float)P;
      a.T_out[o] = (float)T;
      acc += 1.0 - (2.0 * I + a.smooth) / (P + T + a.smooth);
    } else {
      double v = 0.0;
      for (int64_t k = 0; k < nchunk; ++k) v += src[k];
      acc += v;
    }
  }
  acc = block_sum_d(acc, sh);
  if (threadIdx.x == 0) {
    if constexpr (DICE) a.loss[l] = (float)(acc / a.num_masks * a.scale);
    else a.loss[l] = (float)(acc * a.scale / (a.num_masks * (double)a.HtWt));
  }
}

// Gradients, elementwise.  grid (nchunk, C, L*B)
template <bool DICE>
__global__ __launch_bounds__(256) void dense_bwd_kernel(DenseArgs a, int64_t nchunk) {
  const int64_t chunk = blockIdx.x, c = blockIdx.y, lb = blockIdx.z;
  const int64_t b = lb % a.B, l = lb / a.B;
  const int64_t plane = (lb * a.C + c) * a.HW;
  const bool vec = a.dtype == ML_F32 ? (a.HW % 4 == 0) : (a.HW % 8 == 0);
  const int64_t c0 = chunk * kDenseChunk + (int64_t)threadIdx.x * 8;
  // per-plane coefficients (reference: grad_out / (num_masks Ht Wt) in float,
  // times scale; dice: -grad_out / num_masks times scale)
  float coef, I = 0.f, D = 1.f, num = 0.f, invD2 = 0.f;
  if constexpr (DICE) {
    coef = (float)(-(double)a.grad_out[l] / a.num_masks) * a.scale;
    const int64_t o = lb * a.C + c;
    I = a.I_in[o];
    D = a.P_in[o] + a.T_in[o] + a.smooth;
    num = 2.f * I + a.smooth;
    invD2 = 1.f / (D * D);
  } else {
    coef = (float)((double)a.grad_out[l] / (a.num_masks * (double)a.HtWt)) * a.scale;
  }
  float z[kDenseU][8], n[kDenseU][8];
#pragma unroll
  for (int u = 0; u < kDenseU; ++u) {
    const int64_t cell0 = c0 + u * 256 * 8;
    if (cell0 < a.HW) {
      dense_load8(a.logits, a.dtype, plane + cell0, a.HW - cell0, vec, z[u]);
      dense_count8(a, b, c, cell0, n[u]);
    }
  }
#pragma unroll
  for (int u = 0; u < kDenseU; ++u) {
    const int64_t cell0 = c0 + u * 256 * 8;
    if (cell0 >= a.HW) continue;
    float g[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const Sig sg = sig_terms(z[u][k]);
      const float nk = n[u][k];
      if constexpr (DICE) {
        g[k] = coef * ((2.f * nk * D - a.N2 * num) * invD2) * (sg.p * sg.q1);
      } else {
        float mn, mp;
        focal_mods(sg, a.ep, mn, mp);
        const float gm = a.ep.gamma;
        const float gp = -a.ep.ap * nk * mp * (gm * sg.p * sg.cp + sg.q1);
        const float gn = a.ep.an * (a.N2 - nk) * mn * (gm * sg.q1 * sg.cn + sg.p);
        g[k] = (gp + gn) * coef;
      }
    }
    dense_store8(a.grad, a.dtype, plane + cell0, g, a.HW - cell0, vec);
  }
}

int launch_dense(const DenseArgs& a, bool dice, bool backward, hipStream_t st) {
  const int64_t nchunk = ceil_div(a.HW, kDenseChunk);
  if (a.L == 0) return ML_OK;
  if (a.C > 65535 || a.L * a.B > 65535 || nchunk > INT32_MAX)
    return fail(ML_EUNSUPPORTED, "dense loss: grid dimensions out of range");
  const dim3 grid((unsigned)nchunk, (unsigned)a.C, (unsigned)(a.L * a.B));
  const bool work = a.B * a.C > 0 && a.HW > 0;
  ProfScope ps_(dice ? "dice" : "sigmoid_ce", st);
  if (backward) {
    if (!work) return ML_OK;
    if (dice) hipLaunchKernelGGL(dense_bwd_kernel<true>, grid, dim3(256), 0, st, a, nchunk);
    else hipLaunchKernelGGL(dense_bwd_kernel<false>, grid, dim3(256), 0, st, a, nchunk);
    return check_launch("dense backward");
  }
  if (work) {  // no planes: the reduction alone writes zero losses
    if (dice) hipLaunchKernelGGL(dense_fwd_kernel<true>, grid, dim3(256), 0, st, a, nchunk);
    else hipLaunchKernelGGL(dense_fwd_kernel<false>, grid, dim3(256), 0, st, a, nchunk);
    int rc = check_launch("dense forward");
    if (rc) return rc;
  }
  if (dice) hipLaunchKernelGGL(dense_reduce_kernel<true>, dim3((unsigned)a.L), dim3(256), 0, st, a, nchunk);
  else hipLaunchKernelGGL(dense_reduce_kernel<false>, dim3((unsigned)a.L), dim3(256), 0, st, a, nchunk);
  return check_launch("dense reduce");
}

size_t dense_partials_bytes(int64_t L, int64_t B, int64_t C, int64_t HW, bool dice) {
  return (size_t)(L * B * C) * (size_t)ceil_div(HW, kDenseChunk) * (dice ? 3 : 1) * 8;
}

}  // namespace ml
