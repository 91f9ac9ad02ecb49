// Pairwise sigmoid-BCE / dice cost as an MFMA contraction (gfx950).
//
// For one image b, query q and GT column g (label a, count n_g(cell)):
//   bce_num[q,g] = sum_cell A_neg[q,cell] (N2 - n_g) + A_pos[q,cell] n_g
//   I[q,g]       = sum_cell A_p[q,cell] n_g          (intersection)
//   T[q,g]       = sum_cell A_w[q,cell] n_g          (weighted target mass)
// with per-cell planes A_neg = w an mn cn, A_pos = w ap mp cp, A_p = w p, A_w = w.
// An extra "ones" column (n = N2 everywhere) yields the row sums
//   P = sum N2 w p (from the I plane) and S = sum N2 w (from the T plane).
// This is the reference's fused BCE+dice reduction (src/cuda/pw_mask.cu:52-308)
// rewritten as (Q x K)(K x G) products: bce*S = base + Delta of pw_mask.cu:300
// regrouped as sum_{cells} w cn (N2-n) + w cp n (no cancellation between the
// two terms), I and T as pw_mask.cu:270-271, P and S as pw_mask.cu:140-141.
//
// Layout: one workgroup = 4 waves sharing (image, row tile, K-split); each wave
// owns every 4th 32-cell K-step, so the workgroup reads full cache lines of
// every logit row.  Each wave keeps all column tiles of its rows in
// accumulators; the four waves are reduced through LDS in a fixed order and
// one partial per workgroup is written: partials[ks][lb][rtile][3][rows][nslot].
#include "ml_internal.h"

namespace ml {

template <int DT>
struct InTraits;
template <>
struct InTraits<ML_F32> {
  typedef float T;
  static constexpr int kSplit = 3;  // hi/mid/lo bf16 terms: fp32-equivalent products
};
template <>
struct InTraits<ML_BF16> {
  typedef uint16_t T;
  static constexpr int kSplit = 1;
};
template <>
struct InTraits<ML_F16> {
  typedef uint16_t T;
  static constexpr int kSplit = 2;
};

// Load 8 consecutive logits starting at element index i (row-major), zero the
// ones at or beyond `lim` (end of the row).  `vec` = vector load allowed.
template <int DT>
__device__ __forceinline__ void load8(const void* base, int64_t i, int64_t nvalid, bool vec,
                                      float z[8]) {
  if (DT == ML_F32) {
    const float* p = (const float*)base + i;
    if (vec && nvalid >= 8) {
      const float4 v0 = *(const float4*)p;
      const float4 v1 = *(const float4*)(p + 4);
      z[0] = v0.x; z[1] = v0.y; z[2] = v0.z; z[3] = v0.w;
      z[4] = v1.x; z[5] = v1.y; z[6] = v1.z; z[7] = v1.w;
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) z[k] = k < nvalid ? p[k] : 0.f;
    }
  } else {
    const uint16_t* p = (const uint16_t*)base + i;
    if (vec && nvalid >= 8) {
      const uint4 v = *(const uint4*)p;
      const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (DT == ML_BF16) {
          z[2 * k] = bf16_lo(w4[k]);
          z[2 * k + 1] = bf16_hi(w4[k]);
        } else {
          z[2 * k] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w4[k] & 0xFFFF));
          z[2 * k + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w4[k] >> 16));
        }
      }
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint16_t h = k < nvalid ? p[k] : (uint16_t)0;
        z[k] = DT == ML_BF16 ? __uint_as_float(((uint32_t)h) << 16)
                             : (float)__builtin_bit_cast(_Float16, h);
      }
    }
  }
}

// Split 8 fp32 values into NS bf16 terms whose sum reproduces them.
template <int NS>
__device__ __forceinline__ void split_pack(const float v[8], bf16x8_t out[NS]) {
  float rem[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) rem[k] = v[k];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    u32x4_t w;
#pragma unroll
    for (int k = 0; k < 4; ++k) w[k] = pack_bf16x2(rem[2 * k], rem[2 * k + 1]);
    out[s] = __builtin_bit_cast(bf16x8_t, w);
    if (s + 1 < NS) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        rem[2 * k] -= bf16_lo(w[k]);
        rem[2 * k + 1] -= bf16_hi(w[k]);
      }
    }
  }
}

template <int NT, int RT>
struct CostShape {
  static constexpr int kAcc = 3 * RT * NT;  // f32x4 accumulators per lane
};

template <int DT, int RT, int NT, bool CNT>
__global__ __launch_bounds__(256) void cost_kernel(CostArgs a) {
  constexpr int NS = InTraits<DT>::kSplit;
  constexpr int NACC = CostShape<NT, RT>::kAcc;
  __shared__ float red[NACC * 4 * 64];
  __shared__ float red_unw[2 * RT * 16 * 4];

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = lane & 15, g4 = lane >> 4;
  const int64_t lb = blockIdx.z, b = lb % a.B;
  const int64_t q0 = (int64_t)blockIdx.y * (16 * RT);
  const int64_t ks = blockIdx.x;
  const int G = a.ncols[b];
  const int nt_used = (G + 1 + 15) >> 4;
  const bool unw = a.rowsum != nullptr;

  // per-lane column operands.  Tiles below the boundary tile hold real GT
  // columns only (constant operand coefficients); the boundary tile mixes
  // real columns, the ones column (slot G) and padding.
  uint32_t colL[NT];
  const int nt_last = nt_used - 1;
  const int slot_b = nt_last * 16 + r;
  const uint32_t n2pair = pack_bf16x2(a.N2, a.N2);
  const uint32_t base_last = slot_b < G ? 0x3F803F80u : (slot_b == G ? n2pair : 0u);
  const uint32_t coef_last = slot_b < G ? 0x3F803F80u : 0u;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int slot = nt * 16 + r;
    colL[nt] = 0;
    if (slot < G) {
      const int c = a.colmap[b * a.nslot + slot];
      const int act = c + (c >= a.bg ? 1 : 0);
      colL[nt] = (uint32_t)act * 0x10001u;
    }
  }

  f32x4_t acc[3][RT][NT];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[i][rt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float ub[RT], up[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) { ub[rt] = 0.f; up[rt] = 0.f; }

  const ElemParams ep = a.ep;
  const bool vec_ok = DT == ML_F32 ? (a.HW % 4 == 0) : (a.HW % 8 == 0);
  const int64_t nsteps = ceil_div(a.HW, kStep);
  const int64_t stride = a.KS * kWavesCost;

  for (int64_t st = ks * kWavesCost + wave; st < nsteps; st += stride) {
    const int64_t cell0 = st * kStep + g4 * 8;
    const int64_t nvalid = a.HW - cell0;  // may be <= 0 in the tail

    // ---- A planes for RT row tiles
    bf16x8_t A[4][RT][NS];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int64_t q = q0 + rt * 16 + r;
      const bool row_ok = q < a.Q;
      const int64_t qc = row_ok ? q : a.Q - 1;
      float z[8];
      load8<DT>(a.logits, (lb * a.Q + qc) * a.HW + cell0, row_ok ? nvalid : 0, vec_ok, z);
      float v[4][8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const bool ok = row_ok && k < nvalid;
        const Sig s = sig_terms(z[k]);
        const float w = unc_weight(s, ep);
        float mn, mp;
        focal_mods(s, ep, mn, mp);
        const float neg = ep.an * mn * s.cn;
        v[0][k] = ok ? w * neg : 0.f;
        v[1][k] = ok ? w * (ep.ap * mp * s.cp) : 0.f;
        v[2][k] = ok ? w * s.p : 0.f;
        v[3][k] = ok ? w : 0.f;
        if (unw) {
          ub[rt] += ok ? neg : 0.f;
          up[rt] += ok ? s.p : 0.f;
        }
      }
#pragma unroll
      for (int pl = 0; pl < 4; ++pl) split_pack<NS>(v[pl], A[pl][rt]);
    }

    // ---- target operands per column tile, then MFMA
    uint32_t L2[4];
    if (!CNT) {
      const uint4 lv = *(const uint4*)(a.lab16 + b * a.HWp + cell0);
      L2[0] = lv.x; L2[1] = lv.y; L2[2] = lv.z; L2[3] = lv.w;
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if (nt >= nt_used) continue;
      u32x4_t bp, bv;
      const bool last = nt == nt_last;
      if (!CNT) {
        const uint32_t coef = last ? coef_last : 0x3F803F80u;
        const uint32_t base = last ? base_last : 0x3F803F80u;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t m = pk_min_u16(L2[i] ^ colL[nt], 0x00010001u);
          bp[i] = pk_mul_lo_u16(m, coef);
          bv[i] = pk_sub_u16(base, bp[i]);
        }
      } else {
        const int slot = nt * 16 + r;
        const float kB = slot < G ? 1.f : 0.f;
        const float cB = slot == G ? a.N2 : 0.f;
        const uint32_t act = colL[nt] & 0xFFFFu;
        const uint2 cv = *(const uint2*)(a.counts8 + (b * a.GT_total + act) * a.HWp + cell0);
        const uint32_t cw[2] = {cv.x, cv.y};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t word = cw[i >> 1];
          const int sh = (i & 1) * 16;
          const float n0 = (float)((word >> sh) & 0xFF);
          const float n1 = (float)((word >> (sh + 8)) & 0xFF);
          bv[i] = pack_bf16x2(kB * n0 + cB, kB * n1 + cB);
          bp[i] = pack_bf16x2(kB * (a.N2 - n0), kB * (a.N2 - n1));
        }
      }
      const bf16x8_t Bp = __builtin_bit_cast(bf16x8_t, bp);
      const bf16x8_t Bv = __builtin_bit_cast(bf16x8_t, bv);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
        for (int sp = 0; sp < NS; ++sp) {
          acc[0][rt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[0][rt][sp], Bp, acc[0][rt][nt], 0, 0, 0);
          acc[0][rt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[1][rt][sp], Bv, acc[0][rt][nt], 0, 0, 0);
          acc[1][rt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[2][rt][sp], Bv, acc[1][rt][nt], 0, 0, 0);
          acc[2][rt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[3][rt][sp], Bv, acc[2][rt][nt], 0, 0, 0);
        }
      }
    }
  }

  // ---- deterministic cross-wave reduction: wave 3 -> 2 -> 1 -> 0
  for (int w = kWavesCost - 1; w >= 1; --w) {
    if (wave == w) {
      int idx = 0;
#pragma unroll
      for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int e = 0; e < 4; ++e, ++idx) {
              float v = acc[i][rt][nt][e];
              if (w < kWavesCost - 1) v += red[idx * 64 + lane];
              red[idx * 64 + lane] = v;
            }
      if (unw) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          float vb = ub[rt], vp = up[rt];
          if (w < kWavesCost - 1) {
            vb += red_unw[(rt * 2 + 0) * 64 + lane];
            vp += red_unw[(rt * 2 + 1) * 64 + lane];
          }
          red_unw[(rt * 2 + 0) * 64 + lane] = vb;
          red_unw[(rt * 2 + 1) * 64 + lane] = vp;
        }
      }
    }
    __syncthreads();
  }
  if (wave != 0) return;

  const int64_t rows = 16 * RT;
  float* out = a.partials + ((ks * (a.L * a.B) + lb) * a.rtiles + blockIdx.y) * 3 * rows * a.nslot;
  {
    int idx = 0;
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
          for (int e = 0; e < 4; ++e, ++idx) {
            const float v = acc[i][rt][nt][e] + red[idx * 64 + lane];
            const int row = rt * 16 + g4 * 4 + e;
            const int slot = nt * 16 + r;
            out[(i * rows + row) * a.nslot + slot] = v;
          }
  }
  if (unw) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float vb = ub[rt] + red_unw[(rt * 2 + 0) * 64 + lane];
      float vp = up[rt] + red_unw[(rt * 2 + 1) * 64 + lane];
      // lanes r, r+16, r+32, r+48 hold the same row: fixed-order pair sums
      vb += __shfl_xor(vb, 16, 64);
      vp += __shfl_xor(vp, 16, 64);
      vb += __shfl_xor(vb, 32, 64);
      vp += __shfl_xor(vp, 32, 64);
      const int64_t q = q0 + rt * 16 + r;
      if (g4 == 0 && q < a.Q) {
        float* rs = a.rowsum + ((ks * (a.L * a.B) + lb) * a.Qp + q) * 2;
        rs[0] = vb;
        rs[1] = vp;
      }
    }
  }
}

template <int DT, int RT, int NT>
static void launch_one(const CostArgs& a, const Dims& d, hipStream_t st) {
  const dim3 grid((unsigned)d.KS, (unsigned)d.rtiles, (unsigned)d.LB);
  ProfScope ps_("pair_cost", st);
  if (d.counts_mode)
    hipLaunchKernelGGL((cost_kernel<DT, RT, NT, true>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((cost_kernel<DT, RT, NT, false>), grid, dim3(256), 0, st, a);
}

template <int DT>
static int launch_dt(const CostArgs& a, const Dims& d, hipStream_t st) {
  if (d.NT <= 2) launch_one<DT, 1, 2>(a, d, st);
  else if (d.NT <= 4) launch_one<DT, 1, 4>(a, d, st);
  else if (d.NT <= 7) launch_one<DT, 1, 7>(a, d, st);
  else if (d.NT <= 16) launch_one<DT, 1, 16>(a, d, st);
  else return fail(ML_EUNSUPPORTED, "more than 255 GT columns per image are not supported");
  return check_launch("pair_cost");
}

int cost_rt_for(int, int) { return 1; }

int launch_cost(const CostArgs& a, const Dims& d, int dtype, bool, hipStream_t st) {
  switch (dtype) {
    case ML_F32: return launch_dt<ML_F32>(a, d, st);
    case ML_BF16: return launch_dt<ML_BF16>(a, d, st);
    case ML_F16: return launch_dt<ML_F16>(a, d, st);
  }
  return fail(ML_EINVAL, "unsupported mask logits dtype");
}

}  // namespace ml
