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
#include <algorithm>
#include <atomic>

#include "ml_internal.h"

namespace ml {

// Gradient stores are streaming (non-temporal): the gradient is not read
// again by this library, and dirty lines left in the caches would be written
// back while the next cost pass streams the logits, at half its read rate.
__device__ __forceinline__ void store8(void* base, int dt, int64_t i, const float g[8], int64_t nvalid,
                                       bool vec) {
  if (dt == ML_F32) {
    float* p = (float*)base + i;
    if (vec && nvalid >= 8) {
      __builtin_nontemporal_store(f32x4_t{g[0], g[1], g[2], g[3]}, (f32x4_t*)p);
      __builtin_nontemporal_store(f32x4_t{g[4], g[5], g[6], g[7]}, (f32x4_t*)(p + 4));
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
      __builtin_nontemporal_store(u32x4_t{w[0], w[1], w[2], w[3]}, (u32x4_t*)p);
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
  if (a.counts == nullptr) {
    const uint4 lv = *(const uint4*)(a.lab16 + b * a.HWp + cell0);
    const uint32_t w[4] = {lv.x, lv.y, lv.z, lv.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      t[2 * k] = (int64_t)(w[k] & 0xFFFF) == act ? 1.f : 0.f;
      t[2 * k + 1] = (int64_t)(w[k] >> 16) == act ? 1.f : 0.f;
    }
  } else {
    counts8_f(a.counts, a.cw, (b * a.GT_total + act) * a.HWp + cell0, t);
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
template <int EM = 0>
__device__ __forceinline__ float grad_elem(float z, float tk, const ElemParams& ep, float N2,
                                           const RowCoef& r) {
  const Sig s = sig_terms(z);
  const float w = unc_weight_m<EM>(s, ep);
  float mn, mp;
  focal_mods_m<EM>(s, ep, mn, mp);
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
constexpr int64_t kBwdListGrid = 2048;  // workgroups of the matched-list kernel (8 per CU)

// One chunk of kBwdChunk cells of one row.
__device__ __forceinline__ void bwd_chunk(const BwdArgs& a, int64_t row, int64_t chunk) {
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
      // one branch on the modes per 8 cells (wave-uniform), not per cell
      if (default_modes(ep)) {
#pragma unroll
        for (int k = 0; k < 8; ++k) gr[k] = grad_elem<1>(z[u][k], matched ? t[u][k] : 0.f, ep, a.N2, rc);
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) gr[k] = grad_elem(z[u][k], matched ? t[u][k] : 0.f, ep, a.N2, rc);
      }
      store8(a.grad, a.dtype, rbase + cell0, gr, a.HW - cell0, vec);
    }
  }
}

// Every row.  grid: L*B*Q * nchunk
__global__ __launch_bounds__(256) void bwd_mask_chunk_kernel(BwdArgs a, int64_t nchunk) {
  bwd_chunk(a, (int64_t)blockIdx.x / nchunk, (int64_t)blockIdx.x % nchunk);
}

template <int MAXR>
__device__ __forceinline__ void cls_row(const BwdArgs& a, int64_t row);

// Only the rows of the forward's matched list (the rest of the gradient
// already holds zeros); the grid strides over (list entry, chunk) items, so
// its size does not depend on the device-side match count.  With cls_fused,
// the class-logit gradients follow, one row per wave, on the workgroups that
// had the fewest mask items (items are dealt out round robin: the last
// total % grid ones, all of them when the items divide evenly), so they run
// in the mask work's last round instead of in a launch of their own.
__global__ __launch_bounds__(256) void bwd_mask_list_kernel(BwdArgs a, int64_t nchunk) {
  const int64_t rows = a.L * a.B * a.Q;
  const int64_t n = min((int64_t)a.list[0], rows);
  const int64_t total = n * nchunk;
  for (int64_t it = blockIdx.x; it < total; it += gridDim.x) {
    const int64_t row = a.list[1 + it / nchunk];
    if (row >= 0 && row < rows) bwd_chunk(a, row, it % nchunk);
  }
  if (a.cls_fused) {
    constexpr int kWaves = 4;
    const int wave = threadIdx.x >> 6;
    const int64_t G = gridDim.x, extra = total % G;
    const int64_t nlight = extra == 0 ? G : G - extra;
    const int64_t rank = (int64_t)blockIdx.x - (G - nlight);
    if (rank >= 0)
      for (int64_t r0 = rank * kWaves; r0 < rows; r0 += nlight * kWaves)
        if (r0 + wave < rows) cls_row<24>(a, r0 + wave);
  }
}

template <typename I>
__device__ __forceinline__ float cls_in(const void* p, int dt, I i) {
  if (dt == ML_F32) return ((const float*)p)[i];
  const uint16_t h = ((const uint16_t*)p)[i];
  if (dt == ML_BF16) return __uint_as_float(((uint32_t)h) << 16);
  return (float)__builtin_bit_cast(_Float16, h);
}
template <typename I>
__device__ __forceinline__ void cls_out(void* p, int dt, I i, float v) {
  if (dt == ML_F32) {
    ((float*)p)[i] = v;
  } else if (dt == ML_BF16) {
    ((uint16_t*)p)[i] = (uint16_t)(pack_bf16x2(v, 0.f) & 0xFFFF);
  } else {
    ((uint16_t*)p)[i] = __builtin_bit_cast(uint16_t, (_Float16)v);
  }
}

// Class-logit gradient of one (l,b,q) row, on one wave.
constexpr int kClsRegs = 4;   // class rows of up to 256 logits are held in registers
constexpr int kClsBatch = 8;  // longer rows are streamed, kClsBatch loads per lane in flight

// f(c, z) for this lane's classes c = c0, c0 + 64, ... of a row streamed in
// batches (indices clamped into the row, so every load of a batch is issued
// at once)
template <typename F>
__device__ __forceinline__ void for_cls_batched(const BwdArgs& a, int64_t base, int64_t C, F&& f) {
  const int lane = threadIdx.x & 63;
  for (int64_t c0 = lane; c0 < C; c0 += 64 * kClsBatch) {
    float z[kClsBatch];
#pragma unroll
    for (int u = 0; u < kClsBatch; ++u) z[u] = cls_in(a.cls_logits, a.cls_dtype, base + min(c0 + 64 * u, C - 1));
#pragma unroll
    for (int u = 0; u < kClsBatch; ++u)
      if (c0 + 64 * u < C) f(c0 + 64 * u, z[u]);
  }
}

// Softmax-CE gradient of one class row held in registers (NR logits per
// lane, 1 <= C <= 64 NR): every load of the row is issued before the first
// use, then the wave's max, the exp sum and the gradient follow without
// further memory round trips.
template <int NR>
__device__ __forceinline__ void cls_softmax_regs(const BwdArgs& a, int64_t base, int64_t C,
                                                 int64_t tgt, float coeff) {
  const int lane = threadIdx.x & 63;
  // the row's start is wave-uniform, so each access takes a 32-bit offset
  const int es = a.cls_dtype == ML_F32 ? 4 : 2;
  const char* rowp = (const char*)a.cls_logits + base * es;
  char* rowg = (char*)a.grad_cls + base * es;
  const uint32_t last = (uint32_t)C - 1u;
  float zv[NR];
#pragma unroll
  for (int k = 0; k < NR; ++k)
    zv[k] = cls_in(rowp, a.cls_dtype, min((uint32_t)(lane + 64 * k), last));  // clamped into the row
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < NR; ++k)
    if (lane + 64 * k < C) m = fmaxf(m, zv[k]);
  m = wave_max(m);
  float se = 0.f;
#pragma unroll
  for (int k = 0; k < NR; ++k) {
    zv[k] = lane + 64 * k < C ? __expf(zv[k] - m) : 0.f;
    se += zv[k];
  }
  se = wave_sum(se);
  const float inv = se > 0.f ? 1.f / se : 0.f;
#pragma unroll
  for (int k = 0; k < NR; ++k) {
    const uint32_t c = (uint32_t)(lane + 64 * k);
    if (c <= last) cls_out(rowg, a.cls_dtype, c, coeff * (zv[k] * inv - ((int64_t)c == tgt ? 1.f : 0.f)));
  }
}

// MAXR: the largest register form (logits per lane) this caller holds; the
// persistent mask kernel keeps it small so its own registers are not squeezed
template <int MAXR>
__device__ __forceinline__ void cls_row(const BwdArgs& a, int64_t row) {
  const int lane = threadIdx.x & 63;
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
      // rows of up to 64 MAXR logits stay in registers: one round of loads
      if (C <= 64 * kClsRegs) return cls_softmax_regs<kClsRegs>(a, base, C, tgt, coeff);
      if constexpr (MAXR >= 24) {
        if (C <= 64 * 8) return cls_softmax_regs<8>(a, base, C, tgt, coeff);
        if (C <= 64 * 16) return cls_softmax_regs<16>(a, base, C, tgt, coeff);
        if (C <= 64 * 24) return cls_softmax_regs<24>(a, base, C, tgt, coeff);
      }
      float m = -INFINITY;
      for_cls_batched(a, base, C, [&](int64_t, float z) { m = fmaxf(m, z); });
      m = wave_max(m);
      float se = 0.f;
      for_cls_batched(a, base, C, [&](int64_t, float z) { se += __expf(z - m); });
      se = wave_sum(se);
      const float inv = se > 0.f ? 1.f / se : 0.f;
      for_cls_batched(a, base, C, [&](int64_t c, float z) {
        float gv = __expf(z - m) * inv;
        if (c == tgt) gv -= 1.f;
        cls_out(a.grad_cls, a.cls_dtype, base + c, coeff * gv);
      });
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
  for_cls_batched(a, base, C, [&](int64_t c, float z) {
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
  });
}

// one wave per (l,b,q) row; 4 rows per workgroup
__global__ __launch_bounds__(256) void bwd_cls_kernel(BwdArgs a) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row < a.L * a.B * a.Q) cls_row<24>(a, row);
}

// ---- bf16 logits: the per-logit gradient terms from an LDS table ------------
// The mask-logit gradient of a cell with target count tk is
//   mc sf (Fpos tk + Fneg (N2 - tk)) + dc kd Fd (num N2 - 2 D tk)
// with three functions of the logit alone,
//   Fneg = w an mn (g (1-p) cn + p),  Fpos = -w ap mp (g p cp + 1-p),  Fd = w p (1-p),
// which the table holds in float32 (16 bytes per entry) for every bf16 value
// with |z| in [2^-16, 64); |z| < 2^-16 reads the z = 0 entry (relative change
// below 2^-17); |z| >= 64, inf and nan read a NaN marker, and such cells are
// recomputed from the formulas.
constexpr uint32_t kGBase = 111u << 7;          // bf16 magnitude bits of 2^-16
constexpr uint32_t kGOver = 0x4280u;            // bf16 magnitude bits of 64.0
constexpr uint32_t kGN = kGOver - kGBase;       // 2816 regular entries
constexpr uint32_t kGSub = kGBase - 1;          // idx = sat(m - kGSub): 0 = tiny
constexpr uint32_t kGBlock = kGN + 2;           // tiny + regular + overflow slot
constexpr uint32_t kGBytes = 2 * kGBlock * 16;  // both signs: 90176 bytes
constexpr int kLutThreads = 1024;
constexpr int kLutU = 4;                        // 8-cell groups per thread per item
constexpr int64_t kLutChunk = (int64_t)kLutThreads * 8 * kLutU;

__device__ __forceinline__ float4 grad_terms(float z, const ElemParams& ep) {
  const Sig s = sig_terms(z);
  const float w = unc_weight(s, ep);
  float mn, mp;
  focal_mods(s, ep, mn, mp);
  const float g = ep.gamma;
  return make_float4(w * ep.an * mn * (g * s.q1 * s.cn + s.p),
                     -w * ep.ap * mp * (g * s.p * s.cp + s.q1), w * s.p * s.q1, 0.f);
}

__device__ void build_grad_lut(float4* lut, const ElemParams& ep) {
  for (uint32_t e = threadIdx.x; e < 2 * kGBlock; e += blockDim.x) {
    const uint32_t sgn = e >= kGBlock ? 1u : 0u;
    const uint32_t j = e - sgn * kGBlock;
    float4 v;
    if (j <= kGN) {
      const uint32_t mag = j == 0 ? 0u : kGSub + j;
      v = grad_terms(__uint_as_float(((sgn << 15) | mag) << 16), ep);
    } else {
      v = make_float4(__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), 0.f);
    }
    lut[e] = v;
  }
}

// With binary targets (s == 1) a cell needs Fd and only one of Fneg / Fpos:
// two tables of (Fneg, Fd) and (Fpos, Fd) pairs, 8 bytes per entry, picked
// per cell by its target (half the LDS traffic of the 16-byte entries).
// Layout: [target][sign][kGBlock] float2, 90176 bytes in all.
__device__ void build_grad_lut2(float2* lut, const ElemParams& ep) {
  for (uint32_t e = threadIdx.x; e < 2 * kGBlock; e += blockDim.x) {
    const uint32_t sgn = e >= kGBlock ? 1u : 0u;
    const uint32_t j = e - sgn * kGBlock;
    float4 v;
    if (j <= kGN) {
      const uint32_t mag = j == 0 ? 0u : kGSub + j;
      v = grad_terms(__uint_as_float(((sgn << 15) | mag) << 16), ep);
    } else {
      v = make_float4(__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), 0.f);
    }
    lut[e] = make_float2(v.x, v.z);
    lut[2 * kGBlock + e] = make_float2(v.y, v.z);
  }
}

// table indices (sign block included) of the two bf16 logits packed in `u`
__device__ __forceinline__ uint32_t lut_index_pair(uint32_t u) {
  const uint32_t m = u & 0x7FFF7FFFu;
  const uint32_t idx = pk_min_u16(pk_sub_sat_u16(m, kGSub * 0x10001u), (kGN + 1) * 0x10001u);
  return idx + ((u >> 15) & 0x00010001u) * kGBlock;  // negative block (no carry: idx < 2^15)
}

// table entries of the two bf16 logits packed in `u`
__device__ __forceinline__ void lut_pair(uint32_t u, const float4* lut, float4& lo, float4& hi) {
  const uint32_t m = u & 0x7FFF7FFFu;
  uint32_t idx = pk_min_u16(pk_sub_sat_u16(m, kGSub * 0x10001u), (kGN + 1) * 0x10001u);
  idx += ((u >> 15) & 0x00010001u) * kGBlock;  // negative block (no carry: idx < 2^15)
  lo = lut[idx & 0xFFFFu];
  hi = lut[idx >> 16];
}

// One work item of the table kernel: kLutU groups of 8 cells of one row, as
// loaded (raw bf16 logits and raw targets) plus the row's scalars.
struct LutItem {
  int64_t row, cell0;
  int64_t out;           // pred_to_gt of the row
  float S, P, I, T, mc, dc;
  uint4 z[kLutU];        // 8 bf16 logits per group
  uint4 lab[kLutU];      // 8 u16 labels (s == 1), 8 u8 counts in .x/.y or 8 u16 counts (s > 1)
};

template <bool CNT>
__device__ __forceinline__ void lut_load(const BwdArgs& a, int64_t it, int64_t nchunk, bool vec,
                                         LutItem& m) {
  m.row = a.list ? a.list[1 + it / nchunk] : it / nchunk;
  if (m.row < 0 || m.row >= a.L * a.B * a.Q) {  // not a row of this call: skip the item
    m.row = -1;
    return;
  }
  const int64_t lb = m.row / a.Q, l = lb / a.B, b = lb % a.B;
  m.cell0 = (it % nchunk) * kLutChunk + (int64_t)threadIdx.x * 8;
  m.out = a.pred_to_gt[m.row];
  const float* st = a.stats + m.row * ML_STATS;
  m.S = st[ML_STAT_S];
  m.P = st[ML_STAT_P];
  m.I = st[ML_STAT_I];
  m.T = st[ML_STAT_T];
  const float inv_md = a.layer[l * ML_LAYERS + ML_LAYER_INV_MASK_DEN];
  m.mc = a.g_mask[l] * inv_md;
  m.dc = a.g_dice[l] * inv_md;
  const int64_t act = m.out + (m.out >= a.bg ? 1 : 0);
  const int64_t actc = m.out >= 0 && act < a.GT_total ? act : 0;  // a valid slot to read
  const int64_t rbase = m.row * a.HW;
#pragma unroll
  for (int u = 0; u < kLutU; ++u) {
    const int64_t c = m.cell0 + u * kLutThreads * 8;
    m.z[u] = make_uint4(0, 0, 0, 0);
    m.lab[u] = make_uint4(0, 0, 0, 0);
    if (c < a.HW) {
      if (vec) {
        m.z[u] = *(const uint4*)((const uint16_t*)a.logits + rbase + c);
      } else {
        const uint16_t* h = (const uint16_t*)a.logits + rbase + c;
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t lo = c + 2 * k < a.HW ? h[2 * k] : 0u;
          const uint32_t hi = c + 2 * k + 1 < a.HW ? h[2 * k + 1] : 0u;
          w[k] = lo | (hi << 16);
        }
        m.z[u] = make_uint4(w[0], w[1], w[2], w[3]);
      }
      if constexpr (CNT) {
        const int64_t e = (b * a.GT_total + actc) * a.HWp + c;
        if (a.cw == 1) {
          const uint2 cv = *(const uint2*)(a.counts + e);
          m.lab[u] = make_uint4(cv.x, cv.y, 0, 0);
        } else {
          m.lab[u] = *(const uint4*)(a.counts + 2 * e);
        }
      } else {
        m.lab[u] = *(const uint4*)(a.lab16 + b * a.HWp + c);
      }
    }
  }
}

template <bool CNT>
__device__ __forceinline__ void lut_compute_store(const BwdArgs& a, const LutItem& m,
                                                  const float4* lut, bool vec) {
  if (m.row < 0) return;
  const int64_t act = m.out + (m.out >= a.bg ? 1 : 0);
  const bool matched = m.out >= 0 && act < a.GT_total;
  const int64_t rbase = m.row * a.HW;
  if ((!matched && !a.force_masks) || (m.mc == 0.f && m.dc == 0.f)) {
    const float zero[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < kLutU; ++u) {
      const int64_t c = m.cell0 + u * kLutThreads * 8;
      if (c < a.HW) store8(a.grad, ML_BF16, rbase + c, zero, a.HW - c, vec);
    }
    return;
  }
  const RowCoef rc = row_coef(a, m.S, m.P, matched ? m.I : 0.f, matched ? m.T : 0.f, m.mc, m.dc);
  const float cs = rc.mc * rc.sf;
  const float c2 = rc.dc * rc.kd * rc.num * a.N2;
  const float c3 = rc.dc * rc.kd * 2.f * rc.D;
  const uint32_t act32 = matched ? (uint32_t)act : 0xFFFFFFFFu;
#pragma unroll
  for (int u = 0; u < kLutU; ++u) {
    const int64_t c = m.cell0 + u * kLutThreads * 8;
    if (c >= a.HW) continue;
    const uint32_t zw[4] = {m.z[u].x, m.z[u].y, m.z[u].z, m.z[u].w};
    float t[8];
    if constexpr (CNT) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t lw[4] = {m.lab[u].x, m.lab[u].y, m.lab[u].z, m.lab[u].w};
        const uint32_t n = a.cw == 1 ? (lw[k >> 2] >> ((k & 3) * 8)) & 0xFFu
                                     : (lw[k >> 1] >> ((k & 1) * 16)) & 0xFFFFu;
        t[k] = matched ? (float)n : 0.f;
      }
    } else {
      const uint32_t lw[4] = {m.lab[u].x, m.lab[u].y, m.lab[u].z, m.lab[u].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        t[2 * k] = (lw[k] & 0xFFFFu) == act32 ? 1.f : 0.f;
        t[2 * k + 1] = (lw[k] >> 16) == act32 ? 1.f : 0.f;
      }
    }
    float gr[8];
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (CNT) {
        float4 e[2];
        lut_pair(zw[i], lut, e[0], e[1]);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float tk = t[2 * i + h];
          const float g = cs * (e[h].y * tk + e[h].x * fmaxf(a.N2 - tk, 0.f)) + e[h].z * (c2 - c3 * tk);
          bad |= g != g;
          gr[2 * i + h] = g;
        }
      } else {  // tk in {0, 1}, N2 = 1: the (Fneg, Fd) or (Fpos, Fd) table
        const float2* lut2 = (const float2*)lut;
        const uint32_t idx = lut_index_pair(zw[i]);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const bool pos = t[2 * i + h] != 0.f;
          const float2 e = lut2[(h ? idx >> 16 : idx & 0xFFFFu) + (pos ? 2 * kGBlock : 0u)];
          const float g = cs * e.x + e.y * (pos ? c2 - c3 : c2);
          bad |= g != g;
          gr[2 * i + h] = g;
        }
      }
    }
    if (__builtin_expect(bad, 0)) {  // table overflow marker (|z| >= 64, inf, nan): formulas
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float z = (k & 1) ? bf16_hi(zw[k >> 1]) : bf16_lo(zw[k >> 1]);
        if (gr[k] != gr[k]) gr[k] = grad_elem(z, t[k], a.mask_ep, a.N2, rc);
      }
    }
    store8(a.grad, ML_BF16, rbase + c, gr, a.HW - c, vec);
  }
}

// Persistent: one workgroup per CU builds the table, then strides over the
// (row, chunk) items -- the forward's matched rows when `list` is set, every
// row otherwise -- loading item i+1 while item i is computed and stored.
template <bool CNT>
__global__ __launch_bounds__(kLutThreads) void bwd_mask_lut_kernel(BwdArgs a, int64_t nchunk) {
  __shared__ float4 lut[2 * kGBlock];
  const int64_t rows = a.L * a.B * a.Q;
  const int64_t nrows = a.list ? min((int64_t)a.list[0], rows) : rows;
  const int64_t total = nrows * nchunk;
  const bool vec = a.HW % 8 == 0;
  int64_t it = blockIdx.x;
  // the first item's loads (a chain of round trips: row list, row
  // statistics, logits) are issued before the table is built, so their
  // latency overlaps the build
  LutItem cur, nxt;
  if (it < total) lut_load<CNT>(a, it, nchunk, vec, cur);
  if constexpr (CNT) build_grad_lut(lut, a.mask_ep);
  else build_grad_lut2((float2*)lut, a.mask_ep);
  __syncthreads();
  if (it < total) {
    for (; it < total; it += gridDim.x) {
      const int64_t it2 = it + gridDim.x;
      if (it2 < total) lut_load<CNT>(a, it2, nchunk, vec, nxt);
      lut_compute_store<CNT>(a, cur, lut, vec);
      cur = nxt;
    }
  }
  // then the class-logit gradients, one row per wave (no separate launch),
  // on the workgroups that had the fewest mask items (items are dealt out
  // round robin, so those are the last total % grid ones; all of them when
  // the items divide evenly)
  if (a.cls_fused) {
    constexpr int kWaves = kLutThreads / 64;
    const int wave = threadIdx.x >> 6;
    const int64_t G = gridDim.x, extra = total % G;
    const int64_t nlight = extra == 0 ? G : G - extra;
    const int64_t rank = (int64_t)blockIdx.x - (G - nlight);
    if (rank >= 0)
      for (int64_t r0 = rank * kWaves; r0 < rows; r0 += nlight * kWaves)
        if (r0 + wave < rows) cls_row<kClsRegs>(a, r0 + wave);
  }
}

// One persistent workgroup per CU (the 90 KB table allows one per CU).
static int lut_grid() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v < 1)
      v = 256;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

int launch_bwd(const BwdArgs& a, const Dims& d, hipStream_t st) {
  const int64_t rows = d.L * d.B * d.Q;
  bool cls_done = false;  // class-logit gradients fused into the mask kernel
  if (rows > 0 && d.HW > 0) {
    ProfScope ps_("bwd_mask", st);
    if (a.stats && a.dtype == ML_BF16 && g_use_lut) {
      const int64_t nchunk = ceil_div(d.HW, kLutChunk);
      const int64_t grid = std::max<int64_t>(
          1, std::min<int64_t>(std::max(rows * nchunk, ceil_div(rows, kLutThreads / 64)), lut_grid()));
      BwdArgs b = a;
      b.cls_fused = d.C > 0 ? 1 : 0;
      cls_done = true;
      if (d.counts_mode)
        hipLaunchKernelGGL(bwd_mask_lut_kernel<true>, dim3((unsigned)grid), dim3(kLutThreads), 0,
                           st, b, nchunk);
      else
        hipLaunchKernelGGL(bwd_mask_lut_kernel<false>, dim3((unsigned)grid), dim3(kLutThreads), 0,
                           st, b, nchunk);
    } else if (a.stats && a.list) {
      const int64_t nchunk = ceil_div(d.HW, kBwdChunk);
      const int64_t grid = std::max<int64_t>(
          1, std::min<int64_t>(std::max(rows * nchunk, ceil_div(rows, 4)), kBwdListGrid));
      BwdArgs b = a;
      b.cls_fused = d.C > 0 ? 1 : 0;
      cls_done = true;
      hipLaunchKernelGGL(bwd_mask_list_kernel, dim3((unsigned)grid), dim3(256), 0, st, b, nchunk);
    } else if (a.stats) {
      const int64_t nchunk = ceil_div(d.HW, kBwdChunk);
      hipLaunchKernelGGL(bwd_mask_chunk_kernel, dim3((unsigned)(rows * nchunk)), dim3(256), 0, st,
                         a, nchunk);
    } else
      hipLaunchKernelGGL(bwd_mask_kernel, dim3((unsigned)rows), dim3(256), 0, st, a);
    int rc = check_launch("bwd_mask");
    if (rc) return rc;
  }
  if (rows > 0 && d.C > 0 && !cls_done) {
    ProfScope ps_("bwd_cls", st);
    hipLaunchKernelGGL(bwd_cls_kernel, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, st, a);
    return check_launch("bwd_cls");
  }
  return ML_OK;
}

}  // namespace ml
