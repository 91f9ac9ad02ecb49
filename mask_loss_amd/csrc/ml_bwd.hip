// Matched-loss backward.
//
// Mask logits (src/cuda/mask_matching_backward.cu:21-216): for a matched query
// with counts n of its GT (or an unmatched query when unmatched masks are
// forced to empty, n = 0), with detached weights w and normaliser S,
//   d bce / dz  = sigma_s / S * [ -w ap n mp (g p cp + 1-p) + w an (N2-n)+ mn (g (1-p) cn + p) ]
//   d dice / dz = dice_s * w p(1-p) (num N2 - 2 D n) / max(D^2, 1e-20),
//   D = P + T + smooth, num = 2 I + smooth,
// scaled by the upstream layer gradients over the mask denominator.  Other
// rows are zero.  With saved forward statistics (S, P, I, T) every logit is
// read once; without them a first pass recomputes them (the reference's
// two-pass kernel).  Gradients are written in the logits' dtype.
//
// Class logits (src/cuda/mask_matching_backward.cu:218-376): one wave per
// query row, sigmoid one-hot BCE or softmax CE gradients with the reference's
// void / background rules.
#include "ml_internal.h"

namespace ml {

__device__ __forceinline__ void store8(void* base, int dt, int64_t i, const float g[8], int64_t nvalid,
                                       bool vec) {
  if (dt == ML_F32) {
    float* p = (float*)base + i;
    if (vec && nvalid >= 8) {
      *(float4*)p = make_float4(g[0], g[1], g[2], g[3]);
      *(float4*)(p + 4) = make_float4(g[4], g[5], g[6], g[7]);
    } else {
      for (int k = 0; k < 8; ++k)
        if (k < nvalid) p[k] = g[k];
    }
  } else {
    uint16_t* p = (uint16_t*)base + i;
    uint32_t w[4];
    if (dt == ML_BF16) {
#pragma unroll
      for (int k = 0; k < 4; ++k) w[k] = pack_bf16x2(g[2 * k], g[2 * k + 1]);
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
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
}

__device__ __forceinline__ void load8_any(const void* base, int dt, int64_t i, int64_t nvalid,
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
  } else {
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
}

// target count of label `act` for 8 cells starting at cell0
__device__ __forceinline__ void target8(const BwdArgs& a, int64_t b, int64_t act, int64_t cell0,
                                        float t[8]) {
  if (a.counts8 == nullptr) {
    const uint4 lv = *(const uint4*)(a.lab16 + b * a.HWp + cell0);
    const uint32_t w[4] = {lv.x, lv.y, lv.z, lv.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      t[2 * k] = (int64_t)(w[k] & 0xFFFF) == act ? 1.f : 0.f;
      t[2 * k + 1] = (int64_t)(w[k] >> 16) == act ? 1.f : 0.f;
    }
  } else {
    const uint2 cv = *(const uint2*)(a.counts8 + (b * a.GT_total + act) * a.HWp + cell0);
    const uint32_t w[2] = {cv.x, cv.y};
#pragma unroll
    for (int k = 0; k < 8; ++k) t[k] = (float)((w[k >> 2] >> ((k & 3) * 8)) & 0xFF);
  }
}

__device__ float block_sum_256(float v, float* sh) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) sh[wave] = v;
  __syncthreads();
  return ((sh[0] + sh[1]) + (sh[2] + sh[3]));
}

// Per-row coefficients of the mask-logit gradient.
struct RowCoef {
  float mc, dc, sf, D, num, kd;
};

__device__ __forceinline__ RowCoef row_coef(const BwdArgs& a, float S, float P, float I, float T,
                                            float mc, float dc) {
  RowCoef r;
  r.mc = mc;
  r.dc = dc;
  r.sf = a.sigmoid_scale / S;
  r.D = P + T + a.smooth;
  r.num = 2.f * I + a.smooth;
  r.kd = a.dice_scale / fmaxf(r.D * r.D, 1e-20f);
  return r;
}

// d(loss)/dz of one cell with target count tk
__device__ __forceinline__ float grad_elem(float z, float tk, const ElemParams& ep, float N2,
                                           const RowCoef& r) {
  const Sig s = sig_terms(z);
  const float w = unc_weight(s, ep);
  float mn, mp;
  focal_mods(s, ep, mn, mp);
  const float g = ep.gamma;
  const float negc = fmaxf(N2 - tk, 0.f);
  const float gpos = -w * ep.ap * tk * mp * (g * s.p * s.cp + s.q1);
  const float gneg = w * ep.an * negc * mn * (g * s.q1 * s.cn + s.p);
  const float gs = (gpos + gneg) * r.sf;
  const float pp = s.p * s.q1;
  const float gd = (r.num * (w * pp * N2) - 2.f * r.D * (w * pp * tk)) * r.kd;
  return r.mc * gs + r.dc * gd;
}

// Without saved statistics: one workgroup per row, a first pass recomputes
// S, P, I, T (the reference's two-pass kernel).  grid: L*B*Q
__global__ __launch_bounds__(256) void bwd_mask_kernel(BwdArgs a) {
  __shared__ float sh[4 * 4];
  const int64_t row = blockIdx.x;
  const int64_t lb = row / a.Q, l = lb / a.B, b = lb % a.B;
  const int tid = threadIdx.x;
  const int64_t out = a.pred_to_gt[row];
  const int64_t act = out + (out >= a.bg ? 1 : 0);
  const bool matched = out >= 0 && act < a.GT_total;
  const bool vec = a.dtype == ML_F32 ? (a.HW % 4 == 0) : (a.HW % 8 == 0);
  const int64_t rbase = row * a.HW;
  const float inv_md = a.layer[l * ML_LAYERS + ML_LAYER_INV_MASK_DEN];
  const float mc = a.g_mask[l] * inv_md;
  const float dc = a.g_dice[l] * inv_md;
  const int64_t nch = ceil_div(a.HW, 8);

  if ((!matched && !a.force_masks) || (mc == 0.f && dc == 0.f)) {
    const float zero[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t ch = tid; ch < nch; ch += 256)
      store8(a.grad, a.dtype, rbase + ch * 8, zero, a.HW - ch * 8, vec);
    return;
  }
  const ElemParams ep = a.mask_ep;
  float S, P, I, T;
  {
    float sP = 0.f, sT = 0.f, sI = 0.f, sS = 0.f;
    for (int64_t ch = tid; ch < nch; ch += 256) {
      const int64_t cell0 = ch * 8;
      const int64_t nv = a.HW - cell0;
      float z[8], t[8];
      load8_any(a.logits, a.dtype, rbase + cell0, nv, vec, z);
      if (matched) target8(a, b, act, cell0, t);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if (k >= nv) continue;
        const Sig s = sig_terms(z[k]);
        const float w = unc_weight(s, ep);
        const float tk = matched ? t[k] : 0.f;
        sP += w * s.p * a.N2;
        sT += w * tk;
        sI += w * s.p * tk;
        sS += w * a.N2;
      }
    }
    P = block_sum_256(sP, sh);
    T = block_sum_256(sT, sh + 4);
    I = block_sum_256(sI, sh + 8);
    S = block_sum_256(sS, sh + 12);
    if (!a.normalize) S = (float)(a.Ht * a.Wt);
    S = fmaxf(S, kEps);
  }
  const RowCoef rc = row_coef(a, S, P, I, T, mc, dc);
  for (int64_t ch = tid; ch < nch; ch += 256) {
    const int64_t cell0 = ch * 8;
    const int64_t nv = a.HW - cell0;
    float z[8], t[8], gr[8];
    load8_any(a.logits, a.dtype, rbase + cell0, nv, vec, z);
    if (matched) target8(a, b, act, cell0, t);
#pragma unroll
    for (int k = 0; k < 8; ++k) gr[k] = grad_elem(z[k], matched ? t[k] : 0.f, ep, a.N2, rc);
    store8(a.grad, a.dtype, rbase + cell0, gr, nv, vec);
  }
}

// Statistics-driven path: one workgroup per (row, chunk of kBwdChunk cells);
// each thread issues all kBwdU of its logit / label loads before computing,
// so a matched row is spread over many workgroups and its loads overlap.
// grid: L*B*Q * ceil(HW / kBwdChunk)
constexpr int kBwdU = 4;
constexpr int64_t kBwdChunk = 256 * 8 * kBwdU;

__global__ __launch_bounds__(256) void bwd_mask_chunk_kernel(BwdArgs a, int64_t nchunk) {
  const int64_t row = (int64_t)blockIdx.x / nchunk, chunk = (int64_t)blockIdx.x % nchunk;
  const int64_t lb = row / a.Q, l = lb / a.B, b = lb % a.B;
  const int tid = threadIdx.x;
  const int64_t out = a.pred_to_gt[row];
  const int64_t act = out + (out >= a.bg ? 1 : 0);
  const bool matched = out >= 0 && act < a.GT_total;
  const bool vec = a.dtype == ML_F32 ? (a.HW % 4 == 0) : (a.HW % 8 == 0);
  const int64_t rbase = row * a.HW;
  const float inv_md = a.layer[l * ML_LAYERS + ML_LAYER_INV_MASK_DEN];
  const float mc = a.g_mask[l] * inv_md;
  const float dc = a.g_dice[l] * inv_md;
  const int64_t c0 = chunk * kBwdChunk + (int64_t)tid * 8;

  if ((!matched && !a.force_masks) || (mc == 0.f && dc == 0.f)) {
    const float zero[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < kBwdU; ++u) {
      const int64_t cell0 = c0 + u * 256 * 8;
      if (cell0 < a.HW) store8(a.grad, a.dtype, rbase + cell0, zero, a.HW - cell0, vec);
    }
    return;
  }
  const float* st = a.stats + row * ML_STATS;
  const float S = st[ML_STAT_S], P = st[ML_STAT_P];
  const float I = matched ? st[ML_STAT_I] : 0.f;
  const float T = matched ? st[ML_STAT_T] : 0.f;
  const RowCoef rc = row_coef(a, S, P, I, T, mc, dc);
  const ElemParams ep = a.mask_ep;
  float z[kBwdU][8], t[kBwdU][8];
#pragma unroll
  for (int u = 0; u < kBwdU; ++u) {
    const int64_t cell0 = c0 + u * 256 * 8;
    if (cell0 < a.HW) {
      load8_any(a.logits, a.dtype, rbase + cell0, a.HW - cell0, vec, z[u]);
      if (matched) target8(a, b, act, cell0, t[u]);
    }
  }
#pragma unroll
  for (int u = 0; u < kBwdU; ++u) {
    const int64_t cell0 = c0 + u * 256 * 8;
    if (cell0 < a.HW) {
      float gr[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) gr[k] = grad_elem(z[u][k], matched ? t[u][k] : 0.f, ep, a.N2, rc);
      store8(a.grad, a.dtype, rbase + cell0, gr, a.HW - cell0, vec);
    }
  }
}

__device__ __forceinline__ float cls_in(const void* p, int dt, int64_t i) {
  if (dt == ML_F32) return ((const float*)p)[i];
  const uint16_t h = ((const uint16_t*)p)[i];
  if (dt == ML_BF16) return __uint_as_float(((uint32_t)h) << 16);
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ void cls_out(void* p, int dt, int64_t i, float v) {
  if (dt == ML_F32) {
    ((float*)p)[i] = v;
  } else if (dt == ML_BF16) {
    ((uint16_t*)p)[i] = (uint16_t)(pack_bf16x2(v, 0.f) & 0xFFFF);
  } else {
    ((uint16_t*)p)[i] = __builtin_bit_cast(uint16_t, (_Float16)v);
  }
}

// one wave per (l,b,q) row; 4 rows per workgroup
__global__ __launch_bounds__(256) void bwd_cls_kernel(BwdArgs a) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t nrows = a.L * a.B * a.Q;
  if (row >= nrows) return;
  const int64_t lb = row / a.Q, l = lb / a.B, b = lb % a.B;
  const int64_t C = a.C;
  const int64_t base = row * C;
  const int64_t out = a.pred_to_gt[row];
  const int64_t act = out + (out >= a.bg ? 1 : 0);
  const bool matched = out >= 0 && act < a.GT_total;
  const bool has_void = a.void_idx >= 0;
  const bool need_cls = a.force_cls || has_void;
  const float coeff = a.g_cls[l] * (a.cls_scale * a.layer[l * ML_LAYERS + ML_LAYER_INV_CLS_DEN]);
  int64_t y = -1;
  bool zero = (!matched && !need_cls) || coeff == 0.f;
  if (!zero && matched) {
    y = a.cls_targets[b * a.GT_total + act];
    if (y < 0 || y >= C) zero = true;
  }
  if (zero) {
    for (int64_t c = lane; c < C; c += 64) cls_out(a.grad_cls, a.cls_dtype, base + c, 0.f);
    return;
  }
  if (a.use_softmax) {
    if (matched || (a.force_cls && has_void)) {
      const int64_t tgt = matched ? y : a.void_idx;
      float m = -INFINITY;
      for (int64_t c = lane; c < C; c += 64) m = fmaxf(m, cls_in(a.cls_logits, a.cls_dtype, base + c));
      m = wave_max(m);
      float se = 0.f;
      for (int64_t c = lane; c < C; c += 64) se += __expf(cls_in(a.cls_logits, a.cls_dtype, base + c) - m);
      se = wave_sum(se);
      const float inv = se > 0.f ? 1.f / se : 0.f;
      for (int64_t c = lane; c < C; c += 64) {
        float gv = __expf(cls_in(a.cls_logits, a.cls_dtype, base + c) - m) * inv;
        if (c == tgt) gv -= 1.f;
        cls_out(a.grad_cls, a.cls_dtype, base + c, coeff * gv);
      }
    } else {  // has_void only
      for (int64_t c = lane; c < C; c += 64) {
        float gv = 0.f;
        if (c == a.void_idx) {
          const float z = cls_in(a.cls_logits, a.cls_dtype, base + c);
          gv = coeff * (sig_terms(z).p - 1.f);
        }
        cls_out(a.grad_cls, a.cls_dtype, base + c, gv);
      }
    }
    return;
  }
  const ElemParams ep = a.cls_ep;
  const float g = a.cls_gamma;
  const float invC = C > 0 ? 1.f / (float)C : 0.f;
  for (int64_t c = lane; c < C; c += 64) {
    const float z = cls_in(a.cls_logits, a.cls_dtype, base + c);
    const Sig s = sig_terms(z);
    float mn, mp;
    focal_mods(s, ep, mn, mp);
    const float posg = -ep.ap * mp * (g * s.p * s.cp + s.q1);
    const float negg = ep.an * mn * (g * s.q1 * s.cn + s.p);
    const bool is_void = has_void && c == a.void_idx;
    float gv;
    if (matched) {
      gv = coeff * invC * (c == y ? posg : negg);
    } else if (a.force_cls) {
      gv = coeff * invC * (is_void ? posg : negg);
    } else {
      gv = is_void ? coeff * posg : 0.f;
    }
    cls_out(a.grad_cls, a.cls_dtype, base + c, gv);
  }
}

int launch_bwd(const BwdArgs& a, const Dims& d, hipStream_t st) {
  const int64_t rows = d.L * d.B * d.Q;
  if (rows > 0 && d.HW > 0) {
    ProfScope ps_("bwd_mask", st);
    if (a.stats) {
      const int64_t nchunk = ceil_div(d.HW, kBwdChunk);
      hipLaunchKernelGGL(bwd_mask_chunk_kernel, dim3((unsigned)(rows * nchunk)), dim3(256), 0, st,
                         a, nchunk);
    } else
      hipLaunchKernelGGL(bwd_mask_kernel, dim3((unsigned)rows), dim3(256), 0, st, a);
    int rc = check_launch("bwd_mask");
    if (rc) return rc;
  }
  if (rows > 0 && d.C > 0) {
    ProfScope ps_("bwd_cls", st);
    hipLaunchKernelGGL(bwd_cls_kernel, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, st, a);
    return check_launch("bwd_cls");
  }
  return ML_OK;
}

}  // namespace ml
