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
// regrouped as sum_{cells} w cn (N2-n) + w cp n (both terms non-negative, so no
// cancellation), I and T as pw_mask.cu:270-271, P and S as pw_mask.cu:140-141.
//
// Work decomposition: one wave = 16*RT query rows of one image over a
// contiguous range of 32-cell K-steps (K-split index = blockIdx.x); the four
// waves of a workgroup take four consecutive (image, row-tile) tasks.  Each
// image is handled by the kernel instance whose column-tile count NT matches
// its number of non-empty GTs (+1 ones column), so accumulator registers are
// sized to the image, not to the padded GT width.  Every wave writes its own
// partial sums: partials[ks][lb][rtile][3][rows][nslot].
//
// Per-cell planes: bf16 logits take only 65536 values, so for them the four
// planes are read from a per-workgroup LDS table built with the same float32
// formulas (|z| in [2^-9, 64): one entry per bf16 value; |z| < 2^-9: the
// z = 0 entry, which the bf16 planes of such z match to within one rounding
// step; |z| >= 64, inf and nan read a NaN marker, and a wave whose sums come
// out NaN redoes its K-range with the formulas).  Other dtypes
// evaluate the formulas directly and split each plane into NS bf16 terms so
// products keep float32 accuracy.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "ml_internal.h"

namespace ml {

template <int DT>
struct InTraits;
template <>
struct InTraits<ML_F32> {
  static constexpr int kSplit = 3;  // hi/mid/lo bf16 terms: fp32-equivalent products
};
template <>
struct InTraits<ML_BF16> {
  static constexpr int kSplit = 1;
};
template <>
struct InTraits<ML_F16> {
  static constexpr int kSplit = 2;
};

// ---- LUT geometry (bytes): positive block at 0, negative block at 32768 ----
constexpr uint32_t kLutBase = 118u << 7;         // bf16 magnitude bits of 2^-9
constexpr uint32_t kLutOver = 0x4280u;           // bf16 magnitude bits of 64.0
constexpr uint32_t kLutN = kLutOver - kLutBase;  // 1920 regular entries
constexpr uint32_t kLutSub = kLutBase - 1;       // idx = sat(m - kLutSub): 0 = tiny
constexpr uint32_t kLutBlock = kLutN + 2;        // tiny + regular + overflow slot
constexpr uint32_t kLutNegOff = 32768;
constexpr uint32_t kLutBytes = kLutNegOff + kLutBlock * 8;
constexpr int kDepth = 4;  // K-steps of logits in flight per wave

__device__ __forceinline__ uint32_t pk_lshl3_u16(uint32_t a) {
  uint32_t r;
  asm("v_pk_lshlrev_b16 %0, %1, %2" : "=v"(r) : "s"(0x00030003u), "v"(a));
  return r;
}

// (a & m) | (b & ~m) in one v_bfi_b32 (written out, the compiler splits it
// into and / or / bitop3); m wave-uniform (a scalar register)
__device__ __forceinline__ uint32_t bfi32(uint32_t m, uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(m), "v"(a), "v"(b));
  return r;
}

// The four planes of one logit from the float32 formulas (+ the unweighted
// terms of the unmatched-mask penalty).
template <int EM = 0>
__device__ __forceinline__ void planes_formula(float z, const ElemParams& ep, float& neg,
                                               float& pos, float& wp, float& w, float& negu,
                                               float& pu) {
  const Sig s = sig_terms(z);
  w = unc_weight_m<EM>(s, ep);
  float mn, mp;
  focal_mods_m<EM>(s, ep, mn, mp);
  negu = ep.an * mn * s.cn;
  pu = s.p;
  neg = w * negu;
  pos = w * (ep.ap * mp * s.cp);
  wp = w * s.p;
}

// Build the LUT in LDS (all threads of the workgroup).  The overflow slot
// holds NaN so that a wave whose sums come out NaN knows it met |z| >= 64,
// inf or nan (finite table entries cannot produce NaN) and redoes its K-range
// with the formulas.
__device__ void build_lut(unsigned char* lut, const ElemParams& ep) {
  for (uint32_t e = threadIdx.x; e < 2 * kLutBlock; e += blockDim.x) {
    const uint32_t sgn = e >= kLutBlock ? 1u : 0u;
    const uint32_t j = e - sgn * kLutBlock;
    uint2 v;
    if (j <= kLutN) {
      const uint32_t mag = j == 0 ? 0u : kLutSub + j;  // j == 0: |z| < 2^-9 -> z = 0
      const float z = __uint_as_float(((sgn << 15) | mag) << 16);
      float neg, pos, wp, w, nu, pu;
      planes_formula(z, ep, neg, pos, wp, w, nu, pu);
      v.x = pack_bf16x2(neg, pos);
      v.y = pack_bf16x2(wp, w);
    } else {
      v.x = 0x7FC07FC0u;  // NaN marker
      v.y = 0x7FC07FC0u;
    }
    *(uint2*)(lut + sgn * kLutNegOff + j * 8) = v;
  }
}

// 8 consecutive logits of one row as raw words.
template <int DT>
struct Raw8 {
  uint4 w[DT == ML_F32 ? 2 : 1];
};

// `vec`: rows start 16-byte aligned (HW % 4 == 0 for float32, HW % 8 == 0
// otherwise); else the 8 values are read one by one.
template <int DT>
__device__ __forceinline__ void load_raw8(const void* base, int64_t i, Raw8<DT>& r, bool vec) {
  if constexpr (DT == ML_F32) {
    const float* f = (const float*)base + i;
    if (vec) {
      r.w[0] = ((const uint4*)f)[0];
      r.w[1] = ((const uint4*)f)[1];
    } else {
      r.w[0] = make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                          __float_as_uint(f[3]));
      r.w[1] = make_uint4(__float_as_uint(f[4]), __float_as_uint(f[5]), __float_as_uint(f[6]),
                          __float_as_uint(f[7]));
    }
  } else {
    const uint16_t* h = (const uint16_t*)base + i;
    if (vec) {
      r.w[0] = *(const uint4*)h;
    } else {
      r.w[0] = make_uint4((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16),
                          (uint32_t)h[4] | ((uint32_t)h[5] << 16), (uint32_t)h[6] | ((uint32_t)h[7] << 16));
    }
  }
}

template <int DT>
__device__ __forceinline__ void raw_to_f32(const Raw8<DT>& r, float z[8]) {
  if constexpr (DT == ML_F32) {
    const uint32_t u[8] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w,
                           r.w[1].x, r.w[1].y, r.w[1].z, r.w[1].w};
#pragma unroll
    for (int k = 0; k < 8; ++k) z[k] = __uint_as_float(u[k]);
  } else {
    const uint32_t u[4] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (DT == ML_BF16) {
        z[2 * k] = bf16_lo(u[k]);
        z[2 * k + 1] = bf16_hi(u[k]);
      } else {
        z[2 * k] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u[k] & 0xFFFF));
        z[2 * k + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u[k] >> 16));
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

// A planes of one row's 8 cells by formula; with MASK, cells >= nvalid are zero.
template <int DT, int NS, bool MASK>
__device__ __forceinline__ void planes8_formula(const Raw8<DT>& r, const ElemParams& ep,
                                                int64_t nvalid, bool unw, bf16x8_t A[4][NS],
                                                float& ub, float& up) {
  float z[8];
  raw_to_f32<DT>(r, z);
  float v[4][8];
  auto cell = [&](auto em, int k) {
    float neg, pos, wp, w, nu, pu;
    planes_formula<decltype(em)::value>(z[k], ep, neg, pos, wp, w, nu, pu);
    const bool ok = !MASK || k < nvalid;
    v[0][k] = ok ? neg : 0.f;
    v[1][k] = ok ? pos : 0.f;
    v[2][k] = ok ? wp : 0.f;
    v[3][k] = ok ? w : 0.f;
    if (unw) {
      ub += ok ? nu : 0.f;
      up += ok ? pu : 0.f;
    }
  };
  // one branch on the modes per 8 logits (wave-uniform), not per logit
  if (default_modes(ep)) {
#pragma unroll
    for (int k = 0; k < 8; ++k) cell(std::integral_constant<int, 1>(), k);
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) cell(std::integral_constant<int, 0>(), k);
  }
#pragma unroll
  for (int pl = 0; pl < 4; ++pl) split_pack<NS>(v[pl], A[pl]);
}

// Table entries of one row's 8 bf16 cells (LDS reads only; see lut_planes).
__device__ __forceinline__ void lut_lookup8(const uint4& x, const unsigned char* lut, uint2 E[8]) {
  const uint32_t u[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t m = u[i] & 0x7FFF7FFFu;
    const uint32_t idx =
        pk_min_u16(pk_sub_sat_u16(m, kLutSub * 0x10001u), (kLutN + 1) * 0x10001u);
    // sign bits (the negative block's 32 KB offset) merged in with one bitfield insert
    const uint32_t addr = bfi32(0x80008000u, u[i], pk_lshl3_u16(idx));
    E[2 * i] = *(const uint2*)(lut + (addr & 0xFFFFu));
    E[2 * i + 1] = *(const uint2*)(lut + (addr >> 16));
  }
}

// The four A planes from the entries of 8 cells: (neg, pos) and (wp, w) of
// each cell regrouped into per-plane pairs of consecutive cells.
__device__ __forceinline__ void lut_planes(const uint2 E[8], bf16x8_t A[4]) {
  u32x4_t a0, a1, a2, a3;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint2 e0 = E[2 * i], e1 = E[2 * i + 1];
    a0[i] = __builtin_amdgcn_perm(e1.x, e0.x, 0x05040100u);
    a1[i] = __builtin_amdgcn_perm(e1.x, e0.x, 0x07060302u);
    a2[i] = __builtin_amdgcn_perm(e1.y, e0.y, 0x05040100u);
    a3[i] = __builtin_amdgcn_perm(e1.y, e0.y, 0x07060302u);
  }
  A[0] = __builtin_bit_cast(bf16x8_t, a0);
  A[1] = __builtin_bit_cast(bf16x8_t, a1);
  A[2] = __builtin_bit_cast(bf16x8_t, a2);
  A[3] = __builtin_bit_cast(bf16x8_t, a3);
}

// A planes of one row's 8 bf16 cells from the LDS table.
__device__ __forceinline__ void planes8_lut(const uint4& x, const unsigned char* lut,
                                            bf16x8_t A[4]) {
  uint2 E[8];
  lut_lookup8(x, lut, E);
  lut_planes(E, A);
}

// Pacing of the waves of one workgroup that share a CU: the SIMD arbiter
// issues the oldest ready wave first, so with equal work the younger waves
// fall behind and the CU ends the launch at part occupancy.  Every few
// K-steps a wave posts its progress in LDS and drops its issue priority while
// it is ahead of the slowest wave of the workgroup (progress values are
// approximate: no barrier, a stale read only delays the switch).
constexpr int kPaceSlack = 8;  // K-steps ahead of the slowest wave before yielding
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
// The workgroup has at most 16 waves, so lanes 0..15 (one DPP row) hold every
// wave's progress and four DPP swaps within the row give their minimum, with
// no LDS traffic.
__device__ __forceinline__ void pace(int* prog, int k) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  if (lane == 0) prog[wave] = k;
  int v = lane < nw ? prog[lane] : 0x7FFFFFFF;
  v = min(v, dpp_i<0xB1>(v));   // quad_perm [1,0,3,2]
  v = min(v, dpp_i<0x4E>(v));   // quad_perm [2,3,0,1]
  v = min(v, dpp_i<0x141>(v));  // row_half_mirror
  v = min(v, dpp_i<0x140>(v));  // row_mirror
  if (__builtin_amdgcn_readfirstlane(v) + kPaceSlack < k) __builtin_amdgcn_s_setprio(0);
  else __builtin_amdgcn_s_setprio(1);
}

// In-workgroup sum of R consecutive K-splits of one task (R a power of two):
// this wave is split r of its group grp of R waves.  buf: the workgroup's LDS
// exchange area for its writers, 3*RT*NT float4 per lane each; rsbuf: their
// row sums.  buf == null: no reduction.
struct SplitRed {
  f32x4_t* buf = nullptr;
  float2* rsbuf = nullptr;
  int R = 1, r = 0, grp = 0;
};

// One wave's work: 16*RT query rows of task (lb, rtile) over the K-steps of
// split ks of KS; writes the partial sums to `out` ([3][16*RT][16*NT]) and,
// for unweighted penalties, the row sums to `rs` ([16*RT][2]).  TAB:
// per-cell planes from the LDS table (bf16 only); if the sums come out NaN,
// some cell of the K-range hit the table's overflow marker, and the wave
// redoes the range with the formulas before writing.  `setup` (the
// workgroup's table build and barrier) is called exactly once on every path,
// after the first D K-steps of loads are issued, so their latency overlaps it.
// With red.buf, the R waves of the group add their sums in a fixed tree order
// (wave r takes wave r + h for h = R/2, ..., 1; 2 log2(R) barriers for every
// wave of the workgroup) and only wave 0 of the group writes.
template <int DT, int RT, int NT, int CNT, bool TAB, class Setup>
__device__ __forceinline__ void cost_wave(const CostArgs& a, int64_t lb, int64_t rtile,
                                          int64_t ks, int64_t KS, const unsigned char* lut,
                                          float* out, float* rs_out, int* prog, Setup&& setup,
                                          const SplitRed& red = SplitRed(), uint32_t* klut = nullptr) {
  constexpr int NS = InTraits<DT>::kSplit;
  // slot-sum form (classes 1 and 2 on label maps without the table): four
  // planes summed per slot over the cells whose key (the slot of their label's
  // column, or G for cells of no column) is that slot, with one-hot operands
  // only, so each K-step runs the MFMAs of just the column tiles its cells'
  // keys fall in.  klut: this wave's LDS label -> (key | tile bit << 16) table.
  constexpr bool SP = CNT == 0 && !TAB && NT >= 7;
  constexpr int NP = SP ? 4 : 3;
  constexpr int D = TAB ? kDepth : 2;  // K-steps of logits and labels in flight
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, g4 = lane >> 4;
  const ElemParams ep = a.ep;
  const bool unw = !TAB && rs_out != nullptr;
  const int64_t b = lb % a.B;
  const int G = __builtin_amdgcn_readfirstlane(a.ncols[b]);
  const int nt_used = (G + 1 + 15) >> 4;
  const int64_t q0 = rtile * (16 * RT);

  // per-lane column operands: label pair, and the coefficients that turn the
  // match bit into the one-hot (B) and complement (B') bf16 operands.  Real
  // columns: B = 1 on match, B' = 1 elsewhere; ones column (slot G): B = N2,
  // B' = 0; padding: both 0.
  uint32_t colL[NT], coefB[NT], baseB[NT];
  const uint32_t n2pair = pack_bf16x2(a.N2, a.N2);
  if constexpr (!SP) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int slot = nt * 16 + r;
      colL[nt] = 0;
      coefB[nt] = slot < G ? 0x3F803F80u : 0u;
      baseB[nt] = slot < G ? 0x3F803F80u : (slot == G ? n2pair : 0u);
      if (slot < G) {
        const int c = a.colmap[b * a.nslot + slot];
        const int act = c + (c >= a.bg ? 1 : 0);
        colL[nt] = (uint32_t)act * 0x10001u;
      }
    }
  } else {
    // labels (u16, 0xFFFF for none; min(label, 256) indexes the table) ->
    // key: every entry G first, then each column's label its slot (one
    // wave's LDS writes land in issue order; the wait keeps the two rounds
    // apart all the same)
    const uint32_t eG = (uint32_t)G | (1u << (16 + (G >> 4)));
    for (int l = lane; l < 257; l += 64) klut[l] = eG;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    for (int sl = lane; sl < G; sl += 64) {
      const int c = a.colmap[b * a.nslot + sl];
      const int act = c + (c >= a.bg ? 1 : 0);
      if (act >= 0 && act < 256) klut[act] = (uint32_t)sl | (1u << (16 + (sl >> 4)));
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }

  f32x4_t acc[NP][RT][NT];
#pragma unroll
  for (int i = 0; i < NP; ++i)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[i][rt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float ub[RT], up[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    ub[rt] = 0.f;
    up[rt] = 0.f;
  }

  // this wave's K-steps: [s0, s1) of the full steps, plus the tail step
  const int64_t full = a.HW / kStep;
  const int64_t per = ceil_div(full, KS);
  const int64_t s0 = min(full, ks * per);
  const int64_t s1 = min(full, s0 + per);
  const bool has_tail = (a.HW % kStep) != 0 && ks == KS - 1;

  int64_t rowoff[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int64_t q = min(q0 + rt * 16 + r, a.Q - 1);  // rows >= Q compute unused outputs
    rowoff[rt] = (lb * a.Q + q) * a.HW + g4 * 8;
  }
  const uint16_t* labp = a.lab16 + b * a.HWp + g4 * 8;
  const bool vec = DT == ML_F32 ? (a.HW % 4 == 0) : (a.HW % 8 == 0);

  auto mma_step = [&](bf16x8_t (&A)[4][RT][NS], const uint4& lv, int64_t cell0) {
    const uint32_t L2[4] = {lv.x, lv.y, lv.z, lv.w};
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if (nt >= nt_used) continue;
      // CNT == 2 (u16 counts): B = hi + lo with hi = v & 0xFF00 and lo =
      // v & 0xFF, both exact in bf16 (counts and N2 - n reach s*s > 256,
      // which bf16 does not hold exactly), so each product runs twice
      constexpr int NB = CNT == 2 ? 2 : 1;
      u32x4_t bp[NB], bv[NB];
      if constexpr (CNT == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t m = pk_min_u16(L2[i] ^ colL[nt], 0x00010001u);
          bp[0][i] = pk_mul_lo_u16(m, coefB[nt]);
          bv[0][i] = pk_sub_u16(baseB[nt], bp[0][i]);
        }
      } else {
        // real columns: B = n, B' = N2 - n; ones column: B = N2, B' = 0;
        // padding: both 0 (integers: counts never exceed N2)
        const int slot = nt * 16 + r;
        const uint32_t N2i = (uint32_t)a.N2;
        const uint32_t act = colL[nt] & 0xFFFFu;
        uint32_t n[8];
        counts8_u32(a.counts, CNT == 2 ? 2 : 1, (b * a.GT_total + act) * a.HWp + cell0, n);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          uint32_t v[2], p[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            v[h] = slot < G ? n[2 * i + h] : (slot == G ? N2i : 0u);
            p[h] = slot < G ? N2i - n[2 * i + h] : 0u;
          }
          if constexpr (NB == 1) {
            bv[0][i] = pack_bf16x2((float)v[0], (float)v[1]);
            bp[0][i] = pack_bf16x2((float)p[0], (float)p[1]);
          } else {
            bv[0][i] = pack_bf16x2((float)(v[0] & 0xFF00u), (float)(v[1] & 0xFF00u));
            bp[0][i] = pack_bf16x2((float)(p[0] & 0xFF00u), (float)(p[1] & 0xFF00u));
            bv[NB - 1][i] = pack_bf16x2((float)(v[0] & 0xFFu), (float)(v[1] & 0xFFu));
            bp[NB - 1][i] = pack_bf16x2((float)(p[0] & 0xFFu), (float)(p[1] & 0xFFu));
          }
        }
      }
#pragma unroll
      for (int h = 0; h < NB; ++h) {
        const bf16x8_t Bp = __builtin_bit_cast(bf16x8_t, bp[h]);
        const bf16x8_t Bv = __builtin_bit_cast(bf16x8_t, bv[h]);
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
  };

  // slot-sum form: keys of the lane's 8 cells as u16 pairs, and the column
  // tiles any of the K-step's 32 cells falls in (the four lane groups hold
  // different cells; every lane ends with the same mask)
  auto keys_of = [&](const uint4& lv, uint32_t (&kp)[4]) -> uint32_t {
    const uint32_t L2[4] = {lv.x, lv.y, lv.z, lv.w};
    uint32_t e[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      e[2 * i] = klut[min(L2[i] & 0xFFFFu, 256u)];
      e[2 * i + 1] = klut[min(L2[i] >> 16, 256u)];
    }
    uint32_t t = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kp[i] = __builtin_amdgcn_perm(e[2 * i + 1], e[2 * i], 0x0C040C00u);
      t |= e[2 * i] | e[2 * i + 1];
    }
    t >>= 16;
    return __builtin_amdgcn_readlane(t, 0) | __builtin_amdgcn_readlane(t, 16) |
           __builtin_amdgcn_readlane(t, 32) | __builtin_amdgcn_readlane(t, 48);
  };
  auto mma_step_sp = [&](bf16x8_t (&A)[4][RT][NS], const uint32_t (&kp)[4], uint32_t tmask) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if (nt >= nt_used || !((tmask >> nt) & 1u)) continue;
      const uint32_t s2 = (uint32_t)(nt * 16 + r) * 0x10001u;
      u32x4_t bv;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t m = pk_min_u16(kp[i] ^ s2, 0x00010001u);
        bv[i] = pk_sub_u16(0x3F803F80u, pk_mul_lo_u16(m, 0x3F803F80u));
      }
      const bf16x8_t Bv = __builtin_bit_cast(bf16x8_t, bv);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
        for (int sp = 0; sp < NS; ++sp) {
#pragma unroll
          for (int pl = 0; pl < 4; ++pl)
            acc[pl][rt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[pl][rt][sp], Bv, acc[pl][rt][nt], 0, 0, 0);
        }
      }
    }
  };
  // one K-step of either form
  auto mma_any = [&](bf16x8_t (&A)[4][RT][NS], const uint4& lv, int64_t cell0) {
    if constexpr (SP) {
      uint32_t kp[4];
      const uint32_t tm = keys_of(lv, kp);
      mma_step_sp(A, kp, tm);
    } else {
      mma_step(A, lv, cell0);
    }
  };

  // Software pipeline over this wave's nst steps: D steps of logits and
  // labels in flight.  Slot j holds step k + j; it is turned into A operands
  // first and then refilled with step k + j + D (clamped to the last step, so
  // the loads are unconditional and the wait counts stay exact).  Every
  // branch here is wave-uniform.
  // step counters in 32 bits: their compares stay scalar (a wave has at most
  // HW / 32 < 2^31 steps)
  const int nst = (int)(s1 - s0);
  auto planes = [&](const Raw8<DT> (&raw)[RT], bf16x8_t (&A)[4][RT][NS]) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      bf16x8_t T[4][NS];
      if constexpr (TAB) {
        bf16x8_t T1[4];
        planes8_lut(raw[rt].w[0], lut, T1);
#pragma unroll
        for (int pl = 0; pl < 4; ++pl) T[pl][0] = T1[pl];
      } else {
        planes8_formula<DT, NS, false>(raw[rt], ep, 8, unw, T, ub[rt], up[rt]);
      }
#pragma unroll
      for (int pl = 0; pl < 4; ++pl)
#pragma unroll
        for (int sp = 0; sp < NS; ++sp) A[pl][rt][sp] = T[pl][sp];
    }
  };
  if (nst > 0) {
    Raw8<DT> buf[D][RT];
    uint4 lbuf[D];
    // slot j <- step s0 + min(k, nst - 1): logits, labels
    auto fetch_z = [&](int j, int k) {
      const int64_t st = s0 + (k < nst ? k : nst - 1);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) load_raw8<DT>(a.logits, rowoff[rt] + st * kStep, buf[j][rt], vec);
    };
    auto fetch_l = [&](int j, int k) {
      const int64_t st = s0 + (k < nst ? k : nst - 1);
      lbuf[j] = *(const uint4*)(labp + st * kStep);
    };
#pragma unroll
    for (int j = 0; j < D; ++j) {
      fetch_z(j, j);
      fetch_l(j, j);
    }
    setup();
    int k = 0;
    if constexpr (TAB) {
      // table path, software-pipelined one step deep: the LDS reads of step
      // k + 1 are issued before the one-hot operands and MFMAs of step k, so
      // their latency hides behind that work
      uint2 E[RT][8];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) lut_lookup8(buf[0][rt].w[0], lut, E[rt]);
      auto step = [&](int j, int kj, bool refill) {
        bf16x8_t A[4][RT][NS];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          bf16x8_t T1[4];
          lut_planes(E[rt], T1);
#pragma unroll
          for (int pl = 0; pl < 4; ++pl) A[pl][rt][0] = T1[pl];
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) lut_lookup8(buf[(j + 1) % D][rt].w[0], lut, E[rt]);
        __builtin_amdgcn_sched_barrier(0);
        if (refill) fetch_z(j, kj + D);
        mma_step(A, lbuf[j], (s0 + kj) * kStep + g4 * 8);
        __builtin_amdgcn_sched_barrier(0);
        if (refill) fetch_l(j, kj + D);
      };
      for (; k + D <= nst; k += D) {
        if (prog && (k & (2 * D - 1)) == 0) pace(prog, k);
#pragma unroll
        for (int j = 0; j < D; ++j) step(j, k + j, true);
      }
#pragma unroll
      for (int j = 0; j < D - 1; ++j)  // the last nst % D steps
        if (k + j < nst) step(j, k + j, false);
    } else {
      for (; k + D <= nst; k += D) {
        if (prog && (k & (2 * D - 1)) == 0) pace(prog, k);
#pragma unroll
        for (int j = 0; j < D; ++j) {
          // slot-sum form: the key table reads go out before the plane work
          uint32_t kp[4] = {0u, 0u, 0u, 0u}, tm = 0;
          if constexpr (SP) tm = keys_of(lbuf[j], kp);
          bf16x8_t A[4][RT][NS];
          planes(buf[j], A);
          // keep each refill below the last read of its slot, so that it reuses
          // the slot's registers instead of rotating the whole pipeline
          __builtin_amdgcn_sched_barrier(0);
          fetch_z(j, k + j + D);
          if constexpr (SP) mma_step_sp(A, kp, tm);
          else mma_step(A, lbuf[j], (s0 + k + j) * kStep + g4 * 8);
          __builtin_amdgcn_sched_barrier(0);
          fetch_l(j, k + j + D);
        }
      }
#pragma unroll
      for (int j = 0; j < D - 1; ++j) {  // the last nst % D steps
        if (k + j < nst) {
          bf16x8_t A[4][RT][NS];
          planes(buf[j], A);
          mma_any(A, lbuf[j], (s0 + k + j) * kStep + g4 * 8);
        }
      }
    }
  } else {
    setup();
  }

  bool bad = false;
  if constexpr (TAB) {
    // the ones column sees every cell of the row through the w plane, so a
    // NaN marker anywhere in the K-range shows up in acc[2]
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int e = 0; e < 4; ++e) bad |= __builtin_isnan(acc[2][rt][nt][e]);
    bad = __ballot(bad) != 0;
    if (bad) {  // |z| >= 64, inf or nan somewhere in the range: formulas, one step at a time
#pragma unroll
      for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) acc[i][rt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      for (int64_t st = s0; st < s1; ++st) {
        bf16x8_t A[4][RT][NS];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          Raw8<DT> raw;
          load_raw8<DT>(a.logits, rowoff[rt] + st * kStep, raw, vec);
          bf16x8_t T[4][NS];
          planes8_formula<DT, NS, false>(raw, ep, 8, false, T, ub[rt], up[rt]);
#pragma unroll
          for (int pl = 0; pl < 4; ++pl)
#pragma unroll
            for (int sp = 0; sp < NS; ++sp) A[pl][rt][sp] = T[pl][sp];
        }
        mma_step(A, *(const uint4*)(labp + st * kStep), st * kStep + g4 * 8);
      }
    }
  }

  if (has_tail) {  // last partial step: guarded loads, masked planes
    const int64_t st = full;
    const int64_t cell0 = st * kStep + g4 * 8;
    const int64_t nvalid = a.HW - cell0;
    bf16x8_t A[4][RT][NS];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      Raw8<DT> raw;
      uint32_t u[DT == ML_F32 ? 8 : 4];
      const int64_t i0 = rowoff[rt] + st * kStep;
#pragma unroll
      for (int k = 0; k < (DT == ML_F32 ? 8 : 4); ++k) u[k] = 0;
      if constexpr (DT == ML_F32) {
        for (int k = 0; k < 8; ++k)
          if (k < nvalid) u[k] = __float_as_uint(((const float*)a.logits)[i0 + k]);
        raw.w[0] = make_uint4(u[0], u[1], u[2], u[3]);
        raw.w[1] = make_uint4(u[4], u[5], u[6], u[7]);
      } else {
        for (int k = 0; k < 8; ++k)
          if (k < nvalid)
            u[k >> 1] |= (uint32_t)((const uint16_t*)a.logits)[i0 + k] << ((k & 1) * 16);
        raw.w[0] = make_uint4(u[0], u[1], u[2], u[3]);
      }
      bf16x8_t T[4][NS];
      planes8_formula<DT, NS, true>(raw, ep, nvalid, unw, T, ub[rt], up[rt]);
#pragma unroll
      for (int pl = 0; pl < 4; ++pl)
#pragma unroll
        for (int sp = 0; sp < NS; ++sp) A[pl][rt][sp] = T[pl][sp];
    }
    const uint4 lv = *(const uint4*)(labp + st * kStep);
    mma_any(A, lv, cell0);
  }

  if (red.buf) {
    constexpr int TW = NP * RT * NT;  // float4 per lane per writer
    for (int h = red.R >> 1; h >= 1; h >>= 1) {
      const int64_t slot = red.grp * (red.R >> 1) + (red.r & (h - 1));
      if (red.r >= h && red.r < 2 * h) {
        f32x4_t* d = red.buf + slot * TW * 64 + lane;
#pragma unroll
        for (int i = 0; i < NP; ++i)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
              if (nt < nt_used) d[((i * RT + rt) * NT + nt) * 64] = acc[i][rt][nt];
        if (unw) {
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) red.rsbuf[(slot * RT + rt) * 64 + lane] = make_float2(ub[rt], up[rt]);
        }
      }
      __syncthreads();
      if (red.r < h) {
        const f32x4_t* d = red.buf + slot * TW * 64 + lane;
#pragma unroll
        for (int i = 0; i < NP; ++i)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
              if (nt < nt_used) acc[i][rt][nt] += d[((i * RT + rt) * NT + nt) * 64];
        if (unw) {
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            const float2 v = red.rsbuf[(slot * RT + rt) * 64 + lane];
            ub[rt] += v.x;
            up[rt] += v.y;
          }
        }
      }
      __syncthreads();
    }
    if (red.r != 0) return;
  }

  // ---- write this wave's partial sums (only the tiles in use)
  constexpr int rows = 16 * RT, nslot = 16 * NT;
#pragma unroll
  for (int i = 0; i < NP; ++i)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        if (nt >= nt_used) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = rt * 16 + g4 * 4 + e;
          out[(i * rows + row) * nslot + nt * 16 + r] = acc[i][rt][nt][e];
        }
      }
  if (unw) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float vb = ub[rt], vp = up[rt];
      // lanes r, r+16, r+32, r+48 hold the same row: fixed-order pair sums
      vb += __shfl_xor(vb, 16, 64);
      vp += __shfl_xor(vp, 16, 64);
      vb += __shfl_xor(vb, 32, 64);
      vp += __shfl_xor(vp, 32, 64);
      if (g4 == 0) {
        rs_out[(rt * 16 + r) * 2] = vb;
        rs_out[(rt * 16 + r) * 2 + 1] = vp;
      }
    }
  }
}

template <int NT>
constexpr int kClassOf = NT == 2 ? 0 : NT == 7 ? 1 : 2;

// One launch per column-tile class: wave w of the grid takes work item w of
// the class (item = split * n + task index), with the class's tasks, count
// and K-split read from the device schedule.  The grid has
// max(slots, tasks) waves, so every item has a wave.  Where the schedule sets
// R > 1 (classes 1 and 2), items are groups of R waves instead: item u of the
// grid's groups is task u % n at partial u / n, its R waves take R
// consecutive splits of the R * KS-way split and add their sums in LDS
// (n * KS * R <= slots, so the groups fit the grid).
template <int DT, int RT, int NT, int CNT, bool TAB>
__global__ __launch_bounds__(64 * cost_waves(NT, TAB)) void cost_kernel(CostArgs a) {
  constexpr int CI = kClassOf<NT>;
  constexpr int WV = cost_waves(NT, TAB);
  constexpr bool kRed = CI > 0;  // classes whose splits the schedule may group
  constexpr bool SP = CNT == 0 && !TAB && NT >= 7;  // slot-sum form (see cost_wave)
  constexpr int NP = SP ? 4 : 3;                    // planes per partial tile
  __shared__ __align__(16) unsigned char lut_s[TAB ? kLutBytes : 16];
  __shared__ int prog_s[WV];
  __shared__ f32x4_t red_s[kRed ? (WV / 2) * NP * RT * NT * 64 : 1];
  __shared__ uint32_t klut_s[SP ? WV : 1][SP ? 260 : 1];
  __shared__ float2 red_rs[kRed ? (WV / 2) * RT * 64 : 1];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t n = __builtin_amdgcn_readfirstlane(a.sched[CI]);
  const int64_t KS = __builtin_amdgcn_readfirstlane(a.sched[kClasses + CI]);
  const int R = kRed ? __builtin_amdgcn_readfirstlane(a.sched[kSchedRed + CI]) : 1;
  const int64_t total = n * KS;
  // table build + barrier: once per wave, after its first loads are in flight
  auto setup = [&]() {
    if constexpr (TAB) build_lut(lut_s, a.ep);
    __syncthreads();
  };
  constexpr int64_t tile = NP * 16 * RT * 16 * NT;
  uint32_t* klut = SP ? &klut_s[SP ? wave : 0][0] : nullptr;
  if (kRed && R > 1) {
    const int gpw = WV / R;  // groups per workgroup
    const int grp = wave / R, r = wave - grp * R;
    const int64_t u0 = (int64_t)blockIdx.x * gpw;
    if (u0 >= total) return;  // the whole workgroup is idle
    const int64_t u = u0 + grp;
    if (u >= total) {  // an idle group still meets every barrier of the others
      setup();
      for (int h = R >> 1; h >= 1; h >>= 1) {
        __syncthreads();
        __syncthreads();
      }
      return;
    }
    const int64_t i = u % n, kp = u / n;
    const int64_t task = __builtin_amdgcn_readfirstlane(a.sched[kSchedList + CI * a.plan.ntasks + i]);
    const int64_t lb = task / a.rtiles, rtile = task % a.rtiles;
    float* out = a.partials + a.plan.float_base[CI] + u * tile;
    float* rs = a.rowsum ? a.rowsum + (a.plan.slot_base[CI] + u) * (16 * RT) * 2 : nullptr;
    SplitRed red;
    red.buf = red_s;
    red.rsbuf = red_rs;
    red.R = R;
    red.r = r;
    red.grp = grp;
    cost_wave<DT, RT, NT, CNT, TAB>(a, lb, rtile, kp * R + r, KS * R, lut_s, out, rs, nullptr, setup, red,
                                    klut);
    return;
  }
  const int64_t w0 = (int64_t)blockIdx.x * WV;
  if (w0 >= total) return;  // the whole workgroup is idle
  if (threadIdx.x < WV) prog_s[threadIdx.x] = 0;
  const int64_t w = w0 + wave;
  if (w >= total) {
    setup();
    return;
  }
  const int64_t i = w % n, ks = w / n;
  const int64_t task = __builtin_amdgcn_readfirstlane(a.sched[kSchedList + CI * a.plan.ntasks + i]);
  const int64_t lb = task / a.rtiles, rtile = task % a.rtiles;
  float* out = a.partials + a.plan.float_base[CI] + w * tile;
  float* rs = a.rowsum ? a.rowsum + (a.plan.slot_base[CI] + w) * (16 * RT) * 2 : nullptr;
  // pace the waves only where many share the workgroup's CU
  cost_wave<DT, RT, NT, CNT, TAB>(a, lb, rtile, ks, KS, lut_s, out, rs, WV >= 16 ? prog_s : nullptr,
                                  setup, SplitRed(), klut);
}

// ---- bf16 table path with LDS-staged logits (16-row tiles, <= 32 columns) ------
// HBM streams a row best in long runs, while a 16x16x32 MFMA operand spreads
// one K-step over 16 rows (64 bytes each).  So the logits go through LDS: a
// group of 4 K-steps (16 rows x 128 cells, 4 KB) is fetched by four
// global_load_lds_dwordx4, each moving 1 KB as 4 rows x 256 contiguous bytes
// straight into the wave's LDS ring, and read back in the operand layout with
// one ds_read_b128 per K-step.  Instruction i, lane l fetches the 16-byte
// chunk c = (l & 15) ^ R of row R = 4 i + (l >> 4); the hardware stores lane
// l at ring slot 64 i + l = 16 R + (c ^ R), so the reader of K-step s (lane
// (r, g4) wants chunk 4 s + g4 of row r) finds it at slot
// 16 r + ((4 s + g4) ^ r), and the 16 lanes of each read phase touch 16
// different bank groups.  The ring holds kRingGroups groups, so a group's
// fetch is in flight while the previous one is computed, without costing
// registers.  Work items are ordered task-fastest (see row_partials_at), so
// a workgroup's 16 waves stream 16 adjacent row tiles at the same offset.
//
// LDS map of a 16-wave workgroup: positive table block [0, 8 kLutBlock), the
// rings of waves 0 and 1 in the gap before the negative block at kLutNegOff,
// the negative block, then the rings of waves 2..15 (163,072 bytes).
constexpr int kGroupSteps = 4;            // K-steps per group
constexpr uint32_t kGroupBytes = 4096;    // 16 rows x 128 cells x 2 bytes
constexpr int kRingGroups = 2;
constexpr uint32_t kRingBytes = kRingGroups * kGroupBytes;
constexpr uint32_t kDmaWaves = 16;
constexpr uint32_t kLutBlockBytes = kLutBlock * 8;

static_assert(((kLutBlockBytes + 255) & ~255u) + 2 * kRingBytes <= kLutNegOff,
              "two rings fit between the table blocks");
constexpr uint32_t kDmaLds =
    ((kLutNegOff + kLutBlockBytes + 255) & ~255u) + (kDmaWaves - 2) * kRingBytes;
static_assert(kDmaLds <= 160 * 1024, "table and rings fit the LDS of one CU");

// Ring bases are 256-byte aligned, so a reader's address of K-step s is its
// step-0 address with bits 6-7 flipped: (4 s + g4) ^ r = (g4 ^ r) ^ 4 s.
constexpr uint32_t kRingLo = (kLutBlockBytes + 255) & ~255u;
constexpr uint32_t kRingHi = (kLutNegOff + kLutBlockBytes + 255) & ~255u;
__device__ __forceinline__ uint32_t ring_base(int wave) {
  return wave < 2 ? kRingLo + wave * kRingBytes : kRingHi + (wave - 2) * kRingBytes;
}

typedef __attribute__((address_space(3))) void lds_void_t;

// One ds_read_b128 of the wave's ring, complete on return.  Written as
// assembly: the compiler would otherwise wait for every outstanding fetch
// before any LDS read, since it cannot tell which ring slot a
// global_load_lds writes.
__device__ __forceinline__ uint4 ring_read(uint32_t addr) {
  uint4 v;
  asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
  return v;
}

typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u16x2_t as_u16x2(uint32_t v) { return __builtin_bit_cast(u16x2_t, v); }
__device__ __forceinline__ uint32_t as_u32(u16x2_t v) { return __builtin_bit_cast(uint32_t, v); }

// Table byte offsets (sign block included) of the two bf16 logits packed in
// u, as lut_lookup8 computes them, in compiler-visible packed 16-bit ops (no
// inline assembly, so no hazard padding after each one): the clamped index
// times 8 stays below 2^15, so the sign bit ORs in without carry.
__device__ __forceinline__ uint32_t lut_addr_pair(uint32_t u) {
  const u16x2_t m = as_u16x2(u & 0x7FFF7FFFu);
  const u16x2_t idx = __builtin_elementwise_min(
      __builtin_elementwise_sub_sat(m, (u16x2_t){(unsigned short)kLutSub, (unsigned short)kLutSub}),
      (u16x2_t){(unsigned short)(kLutN + 1), (unsigned short)(kLutN + 1)});
  uint32_t addr = (u & 0x80008000u) | as_u32(idx << (u16x2_t){3, 3});
  // kept whole, so its two halves are one mask and one shift of it
  asm("" : "+v"(addr));
  return addr;
}

// Table entries of 8 bf16 cells (as lut_lookup8) read with assembly, and the
// wait for them tied to their registers.  lut_base: the table's LDS address.
__device__ __forceinline__ void lut_lookup8_asm(const uint4& x, uint32_t lut_base, uint64_t E[8]) {
  const uint32_t u[4] = {x.x, x.y, x.z, x.w};
  uint32_t ad[4];  // the four words' chains side by side, then the reads
#pragma unroll
  for (int i = 0; i < 4; ++i) ad[i] = lut_addr_pair(u[i]);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t addr = ad[i];
    asm volatile("ds_read_b64 %0, %1" : "=v"(E[2 * i]) : "v"(lut_base + (addr & 0xFFFFu)) : "memory");
    asm volatile("ds_read_b64 %0, %1" : "=v"(E[2 * i + 1]) : "v"(lut_base + (addr >> 16)) : "memory");
  }
}
// Wait for every outstanding LDS read; E (table entries) and x (ring words
// read earlier) are tied to it, so nothing that uses them moves above it.
__device__ __forceinline__ void lds_wait(uint64_t E[8], uint4& x) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(E[0]), "+v"(E[1]), "+v"(E[2]), "+v"(E[3]), "+v"(E[4]), "+v"(E[5]), "+v"(E[6]),
                 "+v"(E[7]), "+v"(x.x), "+v"(x.y), "+v"(x.z), "+v"(x.w));
}
// Wait for every outstanding LDS read at the end of a pipeline; the
// registers of reads nothing consumes are tied to it, so they stay reserved
// until the data has landed.
__device__ __forceinline__ void lds_drain(uint64_t E[8], uint4 (&x)[2]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(E[0]), "+v"(E[1]), "+v"(E[2]), "+v"(E[3]), "+v"(E[4]), "+v"(E[5]), "+v"(E[6]),
                 "+v"(E[7]), "+v"(x[0].x), "+v"(x[0].y), "+v"(x[0].z), "+v"(x[0].w), "+v"(x[1].x),
                 "+v"(x[1].y), "+v"(x[1].z), "+v"(x[1].w)
               :
               : "memory");
}
// One ds_read_b128 of the ring, not waited for (see lds_wait).
__device__ __forceinline__ uint4 ring_read_async(uint32_t addr) {
  uint4 v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr) : "memory");
  return v;
}
__device__ __forceinline__ void lut_planes64(const uint64_t E64[8], bf16x8_t A[4]) {
  uint2 E[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) E[i] = make_uint2((uint32_t)E64[i], (uint32_t)(E64[i] >> 32));
  lut_planes(E, A);
}
// 16 bytes of labels, loaded with assembly; label_wait<N> waits until at most
// N vector-memory operations issued after it are outstanding.
__device__ __forceinline__ u32x4_t label_load(const void* p) {
  u32x4_t v;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
  return v;
}
template <int N>
__device__ __forceinline__ void label_wait(u32x4_t& v) {
  asm volatile("s_waitcnt vmcnt(%1)" : "+v"(v) : "n"(N));
}
// Drain every vector-memory operation; the label registers are tied to it,
// so loads issued but never used (the pipeline's last ones) keep their
// registers until they have landed (an assembly load's destination would
// otherwise count as free at once and could be reused while it is in flight).
__device__ __forceinline__ void drain_loads(u32x4_t (&l)[4]) {
  asm volatile("s_waitcnt vmcnt(0)" : "+v"(l[0]), "+v"(l[1]), "+v"(l[2]), "+v"(l[3]) : : "memory");
}

template <int NT, class Setup>
__device__ __forceinline__ void cost_wave_dma(const CostArgs& a, int64_t lb, int64_t rtile,
                                              int64_t ks, int64_t KS, const unsigned char* lut,
                                              uint32_t ring, float* out, Setup&& setup) {
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, g4 = lane >> 4;
  const int64_t b = lb % a.B;
  const int G = __builtin_amdgcn_readfirstlane(a.ncols[b]);
  const int nt_used = (G + 1 + 15) >> 4;
  const int64_t q0 = rtile * 16;

  uint32_t colL[NT], coefB[NT], baseB[NT];
  const uint32_t n2pair = pack_bf16x2(a.N2, a.N2);
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int slot = nt * 16 + r;
    colL[nt] = 0;
    coefB[nt] = slot < G ? 0x3F803F80u : 0u;
    baseB[nt] = slot < G ? 0x3F803F80u : (slot == G ? n2pair : 0u);
    if (slot < G) {
      const int c = a.colmap[b * a.nslot + slot];
      const int act = c + (c >= a.bg ? 1 : 0);
      colL[nt] = (uint32_t)act * 0x10001u;
    }
  }
  f32x4_t acc[3][NT];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[i][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // this wave's K-steps: whole groups [g0, g1) of the row's full K-steps
  const int64_t full = a.HW / kStep;
  const int64_t ngr = ceil_div(full, kGroupSteps);
  const int64_t gper = ceil_div(ngr, KS);
  const int64_t g0 = min(ngr, ks * gper), g1 = min(ngr, g0 + gper);
  const int64_t s0 = g0 * kGroupSteps;
  const int nst = (int)(min(full, g1 * kGroupSteps) - s0);
  const bool has_tail = (a.HW % kStep) != 0 && ks == KS - 1;

  // fetch sources: instruction i of a group reads row R = 4 i + (lane >> 4)
  // (clamped to the last query) at chunk (lane & 15) ^ R; element offsets
  // from zrow0 stay below 2^31 (host check)
  const uint16_t* zrow0 = (const uint16_t*)a.logits + (lb * a.Q + q0) * a.HW;
  const uint32_t HW32 = (uint32_t)a.HW, qlast = (uint32_t)(a.Q - 1 - q0);
  auto fetch_group = [&](int slot, int64_t g) {  // g in [g0, g1)
    const uint32_t cell0 = (uint32_t)(g * (kGroupSteps * kStep));
    const bool edge = cell0 + kGroupSteps * kStep > HW32;  // wave-uniform
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t R = 4u * i + g4;
      uint32_t cell = cell0 + 8u * (((uint32_t)lane & 15u) ^ R);
      if (edge) cell = min(cell, HW32 - 8u);  // past the row end: its last chunk (never used)
      const uint32_t off = min(R, qlast) * HW32 + cell;
      __builtin_amdgcn_global_load_lds((const void*)(zrow0 + off),
                                       (lds_void_t*)(size_t)(ring + slot * kGroupBytes + i * 1024), 16, 0, 0);
    }
  };
  // reader of K-step s: ring + slot * kGroupBytes + 16 (16 r + ((4 s + g4) ^ r))
  const uint32_t rd = ring + 16u * (16u * r + ((uint32_t)g4 ^ (uint32_t)r));
  auto step_addr = [&](int t) {
    const int s = t & (kGroupSteps - 1), slot = (t / kGroupSteps) & (kRingGroups - 1);
    return (rd ^ (64u * s)) + slot * kGroupBytes;
  };
  const uint16_t* labp = a.lab16 + b * a.HWp + g4 * 8;
  u32x4_t lbuf[kGroupSteps];
  auto fetch_l = [&](int j, int t) {
    const int64_t st = s0 + (t < nst ? t : nst - 1);
    lbuf[j] = label_load(labp + st * kStep);
  };

  auto mma = [&](const bf16x8_t (&A)[4], const uint4& lv) {
    const uint32_t L2[4] = {lv.x, lv.y, lv.z, lv.w};
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if (nt >= nt_used) continue;
      u32x4_t bp, bv;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t m = pk_min_u16(L2[i] ^ colL[nt], 0x00010001u);
        bp[i] = pk_mul_lo_u16(m, coefB[nt]);
        bv[i] = pk_sub_u16(baseB[nt], bp[i]);
      }
      const bf16x8_t Bp = __builtin_bit_cast(bf16x8_t, bp);
      const bf16x8_t Bv = __builtin_bit_cast(bf16x8_t, bv);
      acc[0][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[0], Bp, acc[0][nt], 0, 0, 0);
      acc[0][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[1], Bv, acc[0][nt], 0, 0, 0);
      acc[1][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[2], Bv, acc[1][nt], 0, 0, 0);
      acc[2][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[3], Bv, acc[2][nt], 0, 0, 0);
    }
  };

  // Every load of the pipeline is issued in this order, so the vmcnt waits
  // below are exact: labels of steps 0..3, groups 0 and 1; then per step t:
  // [refill of this group's slot (s = 3)] [label of step t + 4].  The label
  // of step t is then followed by exactly (near the start: at least) 7 later
  // loads when it is used, and a group's fetch by at least 2 when its first
  // step is read from the ring (two steps before that step).  LDS reads run
  // two steps ahead for the ring and one for the table: step t waits for
  // both (lds_wait), then issues the ring read of step t + 2 and the table
  // reads of step t + 1.
  if (nst > 0) {
    const int ngl = (int)(g1 - g0);
    const uint32_t lut_base = (uint32_t)(size_t)(lds_void_t*)lut;
#pragma unroll
    for (int j = 0; j < kGroupSteps; ++j) fetch_l(j, j);
    fetch_group(0, g0);
    fetch_group(1, g0 + (ngl > 1 ? 1 : 0));
    setup();
    __builtin_amdgcn_s_waitcnt(0x0F74);  // vmcnt(4): group 0 landed (group 1 may be in flight)
    uint64_t E[8];
    uint4 xr[2];  // ring words of steps t + 1 (xr[(t + 1) & 1]) and t + 2
    lut_lookup8_asm(ring_read(step_addr(0)), lut_base, E);
    xr[1] = nst > 1 ? ring_read_async(step_addr(1)) : make_uint4(0u, 0u, 0u, 0u);
    for (int t0 = 0; t0 < nst; t0 += kGroupSteps) {
#pragma unroll
      for (int s = 0; s < kGroupSteps; ++s) {  // s compile-time: lbuf and xr stay in registers
        const int t = t0 + s;
        if (t < nst) {
          uint4& xn = xr[(s + 1) & 1];  // step t + 1
          uint4& xnn = xr[s & 1];       // step t + 2
          lds_wait(E, xn);
          bf16x8_t A[4];
          lut_planes64(E, A);
          if (t + 1 < nst) lut_lookup8_asm(xn, lut_base, E);
          if (t + 2 < nst) {
            if (s == kGroupSteps - 2)  // step t + 2 opens the next group: its fetch has landed
              __builtin_amdgcn_s_waitcnt(0x0F72);  // when at most 2 later loads are pending
            xnn = ring_read_async(step_addr(t + 2));
          }
          if (s == kGroupSteps - 1) {  // every step of this slot is read: refill it two groups on
            const int k = t0 / kGroupSteps;
            fetch_group(k & (kRingGroups - 1), g0 + min(k + kRingGroups, ngl - 1));
          }
          label_wait<7>(lbuf[s]);
          __builtin_amdgcn_sched_barrier(0);
          mma(A, __builtin_bit_cast(uint4, lbuf[s]));
          __builtin_amdgcn_sched_barrier(0);
          fetch_l(s, t + kGroupSteps);
        }
      }
    }
    drain_loads(lbuf);  // also: no fetch may land in LDS after the wave ends
  } else {
    setup();
  }

  // |z| >= 64, inf or nan somewhere in the range (the ones column's w plane
  // sees every cell): formulas, one step at a time
  bool bad = false;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int e = 0; e < 4; ++e) bad |= __builtin_isnan(acc[2][nt][e]);
  bad = __ballot(bad) != 0;
  const ElemParams ep = a.ep;
  const int64_t rowoff = (lb * a.Q + min(q0 + r, a.Q - 1)) * a.HW + g4 * 8;
  auto formula_step = [&](int64_t st, int64_t nvalid) {
    Raw8<ML_BF16> raw;
    const uint16_t* zp = (const uint16_t*)a.logits + rowoff + st * kStep;
    uint32_t u[4] = {0u, 0u, 0u, 0u};
    for (int k = 0; k < 8; ++k)
      if (k < nvalid) u[k >> 1] |= (uint32_t)zp[k] << ((k & 1) * 16);
    raw.w[0] = make_uint4(u[0], u[1], u[2], u[3]);
    bf16x8_t T[4][1];
    float ub = 0.f, up = 0.f;
    if (nvalid >= 8) planes8_formula<ML_BF16, 1, false>(raw, ep, 8, false, T, ub, up);
    else planes8_formula<ML_BF16, 1, true>(raw, ep, nvalid, false, T, ub, up);
    const bf16x8_t A[4] = {T[0][0], T[1][0], T[2][0], T[3][0]};
    mma(A, *(const uint4*)(labp + st * kStep));
  };
  if (bad) {
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[i][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int64_t st = s0; st < s0 + nst; ++st) formula_step(st, 8);
  }
  if (has_tail) formula_step(full, a.HW - (full * kStep + g4 * 8));

  constexpr int nslot = 16 * NT;
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if (nt >= nt_used) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) out[(i * 16 + g4 * 4 + e) * nslot + nt * 16 + r] = acc[i][nt][e];
    }
}

template <int NT>
__global__ __launch_bounds__(64 * kDmaWaves) void cost_dma_kernel(CostArgs a) {
  constexpr int CI = kClassOf<NT>;
  __shared__ __align__(16) unsigned char lds[kDmaLds];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t n = __builtin_amdgcn_readfirstlane(a.sched[CI]);
  const int64_t KS = __builtin_amdgcn_readfirstlane(a.sched[kClasses + CI]);
  const int64_t total = n * KS;
  const int64_t w0 = (int64_t)blockIdx.x * kDmaWaves;
  if (w0 >= total) return;  // the whole workgroup is idle
  auto setup = [&]() {
    build_lut(lds, a.ep);
    __syncthreads();
  };
  const int64_t w = w0 + wave;
  if (w >= total) {
    setup();
    return;
  }
  const int64_t i = w % n, ks = w / n;
  const int64_t task = __builtin_amdgcn_readfirstlane(a.sched[kSchedList + CI * a.plan.ntasks + i]);
  const int64_t lb = task / a.rtiles, rtile = task % a.rtiles;
  constexpr int64_t tile = 3 * 16 * 16 * NT;
  float* out = a.partials + a.plan.float_base[CI] + w * tile;
  const uint32_t ring = (uint32_t)(size_t)(lds_void_t*)lds + ring_base(wave);
  cost_wave_dma<NT>(a, lb, rtile, ks, KS, lds, ring, out, setup);
}

// ---- class 0 as row-tile pairs: 32x32x16 products ------------------------------
// One wave takes 32 query rows (row tiles 2k and 2k + 1 of one image) and the
// 32 column slots of class 0 over its K-range, in K-steps of 16 cells:
// lane (r = lane & 31, h = lane >> 5) holds cells 8 h .. 8 h + 7 of the step
// for query row r (A operand) and for column slot r (B operand), and its
// accumulators hold column r at rows 8 (v / 4) + 4 h + v % 4 of register v.
// Against the 16-row kernel, one B operand (the label compare) now serves 32
// query rows, which halves the vector-ALU work of the column side per logit.
// Logits go through the same LDS ring: a group is 4 K-steps (64 cells) of the
// 32 rows, 128 bytes per row; instruction i of a group fetch has lane l load
// row R = 8 i + (l >> 3) at chunk c = (l & 7) ^ (R & 7) into slot
// 8 R + (c ^ (R & 7)), so the 8 lanes of each ds_read_b128 phase (8
// consecutive rows, one chunk) touch 8 different bank groups.
//
// A workgroup is 4 pairs x 4 adjacent K-splits (wave = 4 pair + split): the
// four splits of a pair are summed in LDS at the end, in the fixed order
// (s0 + s2) + (s1 + s3), and only that sum is written, so the partial sums
// that reach memory (and the finalize's reads of them) are a quarter of one
// tile per wave.  The schedule's class-0 split count is the number of such
// quads, KSq; the kernel runs 4 KSq K-ranges.
constexpr int kPairStep = 16;                               // cells per K-step
constexpr int kPairGroupCells = kGroupSteps * kPairStep;    // 64 cells x 32 rows = 4 KB
constexpr int64_t kPairTile = 3 * 32 * 32;                  // partial tile (floats)
static_assert(kPairGroupCells * 32 * 2 == (int)kGroupBytes, "a pair group fills one ring slot");

template <class Setup>
__device__ __forceinline__ void cost_wave_pair(const CostArgs& a, int64_t lb, int64_t q0, int64_t ks,
                                               int64_t KS, const unsigned char* lut, uint32_t ring,
                                               f32x16_t (&acc)[3], Setup&& setup) {
  const int lane = threadIdx.x & 63;
  const int r = lane & 31, h = lane >> 5;
  const int64_t b = lb % a.B;
  const int G = __builtin_amdgcn_readfirstlane(a.ncols[b]);

  // column operand of slot r (see cost_wave): real columns compare labels,
  // slot G is the ones column, the rest is padding
  uint32_t colL = 0;
  const uint32_t coefB = r < G ? 0x3F803F80u : 0u;
  const uint32_t baseB = r < G ? 0x3F803F80u : (r == G ? pack_bf16x2(a.N2, a.N2) : 0u);
  if (r < G) {
    const int c = a.colmap[b * a.nslot + r];
    colL = (uint32_t)(c + (c >= a.bg ? 1 : 0)) * 0x10001u;
  }
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][e] = 0.f;

  const int64_t full = a.HW / kPairStep;
  const int64_t ngr = ceil_div(full, kGroupSteps);
  const int64_t gper = ceil_div(ngr, KS);
  const int64_t g0 = min(ngr, ks * gper), g1 = min(ngr, g0 + gper);
  const int64_t s0 = g0 * kGroupSteps;
  const int nst = (int)(min(full, g1 * kGroupSteps) - s0);
  const bool has_tail = (a.HW % kPairStep) != 0 && ks == KS - 1;

  // fetch sources: rows past the last query read the last query's row
  // (never used); element offsets from zrow0 stay below 2^31 (host check)
  const uint16_t* zrow0 = (const uint16_t*)a.logits + (lb * a.Q + q0) * a.HW;
  const uint32_t HW32 = (uint32_t)a.HW, qlast = (uint32_t)(a.Q - 1 - q0);
  auto fetch_group = [&](int slot, int64_t g) {  // g in [g0, g1)
    const uint32_t cell0 = (uint32_t)(g * kPairGroupCells);
    const bool edge = cell0 + kPairGroupCells > HW32;  // wave-uniform
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t R = 8u * i + ((uint32_t)lane >> 3);
      uint32_t cell = cell0 + 8u * (((uint32_t)lane & 7u) ^ (R & 7u));
      if (edge) cell = min(cell, HW32 - 8u);  // past the row end: its last chunk (never used)
      const uint32_t off = min(R, qlast) * HW32 + cell;
      __builtin_amdgcn_global_load_lds((const void*)(zrow0 + off),
                                       (lds_void_t*)(size_t)(ring + slot * kGroupBytes + i * 1024), 16, 0, 0);
    }
  };
  // reader of K-step s: ring + slot * kGroupBytes + 128 r + 16 ((2 s + h) ^ (r & 7));
  // the ring is 256-byte aligned, so that is the step-0 address with bits 5-6
  // flipped by 2 s
  const uint32_t rd = ring + 128u * r + 16u * ((uint32_t)h ^ ((uint32_t)r & 7u));
  auto step_addr = [&](int t) {
    const int s = t & (kGroupSteps - 1), slot = (t / kGroupSteps) & (kRingGroups - 1);
    return (rd ^ (32u * s)) + slot * kGroupBytes;
  };
  const uint16_t* labp = a.lab16 + b * a.HWp + h * 8;
  u32x4_t lbuf[kGroupSteps];
  auto fetch_l = [&](int j, int t) {
    const int64_t st = s0 + (t < nst ? t : nst - 1);
    lbuf[j] = label_load(labp + st * kPairStep);
  };

  auto mma = [&](const bf16x8_t (&A)[4], const uint4& lv) {
    const uint32_t L2[4] = {lv.x, lv.y, lv.z, lv.w};
    u32x4_t bp, bv;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t m = pk_min_u16(L2[i] ^ colL, 0x00010001u);
      bp[i] = pk_mul_lo_u16(m, coefB);
      bv[i] = pk_sub_u16(baseB, bp[i]);
    }
    const bf16x8_t Bp = __builtin_bit_cast(bf16x8_t, bp);
    const bf16x8_t Bv = __builtin_bit_cast(bf16x8_t, bv);
    acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[0], Bp, acc[0], 0, 0, 0);
    acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[2], Bv, acc[1], 0, 0, 0);
    acc[2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[3], Bv, acc[2], 0, 0, 0);
    acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[1], Bv, acc[0], 0, 0, 0);
  };

  // The pipeline and its wait counts are those of cost_wave_dma: per K-step
  // one label load, per group one 4-instruction fetch, in the same order.
  if (nst > 0) {
    const int ngl = (int)(g1 - g0);
    const uint32_t lut_base = (uint32_t)(size_t)(lds_void_t*)lut;
#pragma unroll
    for (int j = 0; j < kGroupSteps; ++j) fetch_l(j, j);
    fetch_group(0, g0);
    fetch_group(1, g0 + (ngl > 1 ? 1 : 0));
    setup();
    __builtin_amdgcn_s_waitcnt(0x0F74);  // vmcnt(4): group 0 landed (group 1 may be in flight)
    uint64_t E[8];
    uint4 xr[2];  // ring words of steps t + 1 (xr[(t + 1) & 1]) and t + 2
    lut_lookup8_asm(ring_read(step_addr(0)), lut_base, E);
    xr[1] = nst > 1 ? ring_read_async(step_addr(1)) : make_uint4(0u, 0u, 0u, 0u);
    for (int t0 = 0; t0 < nst; t0 += kGroupSteps) {
#pragma unroll
      for (int s = 0; s < kGroupSteps; ++s) {  // s compile-time: lbuf and xr stay in registers
        const int t = t0 + s;
        if (t < nst) {
          uint4& xn = xr[(s + 1) & 1];  // step t + 1
          uint4& xnn = xr[s & 1];       // step t + 2
          lds_wait(E, xn);
          bf16x8_t A[4];
          lut_planes64(E, A);
          // E is consumed above the next lookups, which then reuse its
          // registers.  Past the last step the lookups and ring reads still
          // run (on stale ring words: table addresses stay in the table, ring
          // addresses in the ring), so no value depends on the step count;
          // lds_drain below waits for them.
          __builtin_amdgcn_sched_barrier(0);
          lut_lookup8_asm(xn, lut_base, E);
          if (s == kGroupSteps - 2)  // step t + 2 opens the next group: its fetch has landed
            __builtin_amdgcn_s_waitcnt(0x0F72);  // when at most 2 later loads are pending
          xnn = ring_read_async(step_addr(t + 2));
          if (s == kGroupSteps - 1) {  // every step of this slot is read: refill it two groups on
            const int k = t0 / kGroupSteps;
            fetch_group(k & (kRingGroups - 1), g0 + min(k + kRingGroups, ngl - 1));
          }
          label_wait<7>(lbuf[s]);
          __builtin_amdgcn_sched_barrier(0);
          mma(A, __builtin_bit_cast(uint4, lbuf[s]));
          __builtin_amdgcn_sched_barrier(0);
          fetch_l(s, t + kGroupSteps);
        }
      }
    }
    lds_drain(E, xr);
    drain_loads(lbuf);  // also: no fetch may land in LDS after the wave ends
  } else {
    setup();
  }

  // |z| >= 64, inf or nan somewhere in the range: formulas, one step at a time
  bool bad = false;
#pragma unroll
  for (int e = 0; e < 16; ++e) bad |= __builtin_isnan(acc[2][e]);
  bad = __ballot(bad) != 0;
  const ElemParams ep = a.ep;
  const int64_t rowoff = (lb * a.Q + min(q0 + r, a.Q - 1)) * a.HW + h * 8;
  auto formula_step = [&](int64_t st, int64_t nvalid) {
    Raw8<ML_BF16> raw;
    const uint16_t* zp = (const uint16_t*)a.logits + rowoff + st * kPairStep;
    uint32_t u[4] = {0u, 0u, 0u, 0u};
    for (int k = 0; k < 8; ++k)
      if (k < nvalid) u[k >> 1] |= (uint32_t)zp[k] << ((k & 1) * 16);
    raw.w[0] = make_uint4(u[0], u[1], u[2], u[3]);
    bf16x8_t T[4][1];
    float ub = 0.f, up = 0.f;
    if (nvalid >= 8) planes8_formula<ML_BF16, 1, false>(raw, ep, 8, false, T, ub, up);
    else planes8_formula<ML_BF16, 1, true>(raw, ep, nvalid, false, T, ub, up);
    const bf16x8_t A[4] = {T[0][0], T[1][0], T[2][0], T[3][0]};
    mma(A, *(const uint4*)(labp + st * kPairStep));
  };
  if (bad) {
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][e] = 0.f;
    for (int64_t st = s0; st < s0 + nst; ++st) formula_step(st, 8);
  }
  if (has_tail) formula_step(full, a.HW - (full * kPairStep + h * 8));
}

// One wave's accumulators in LDS (12 KB): 4 consecutive registers per lane
// as one 16-byte word, consecutive lanes at consecutive words.
__device__ __forceinline__ void acc_to_lds(float* buf, const f32x16_t (&acc)[3], int lane) {
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int v4 = 0; v4 < 4; ++v4)
      *(f32x4_t*)(buf + ((i * 4 + v4) * 64 + lane) * 4) =
          f32x4_t{acc[i][4 * v4], acc[i][4 * v4 + 1], acc[i][4 * v4 + 2], acc[i][4 * v4 + 3]};
}
__device__ __forceinline__ void acc_add_lds(f32x16_t (&acc)[3], const float* buf, int lane) {
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int v4 = 0; v4 < 4; ++v4) {
      const f32x4_t x = *(const f32x4_t*)(buf + ((i * 4 + v4) * 64 + lane) * 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[i][4 * v4 + e] += x[e];
    }
}

__global__ __launch_bounds__(64 * kDmaWaves) void cost_pair_kernel(CostArgs a) {
  __shared__ __align__(16) unsigned char lds[kDmaLds];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t n = __builtin_amdgcn_readfirstlane(a.sched[0]);
  const int64_t KSq = __builtin_amdgcn_readfirstlane(a.sched[kClasses]);
  const int64_t rt = a.rtiles, prt = (rt + 1) >> 1;
  const int64_t np = (n / rt) * prt;  // class 0 holds whole images
  const int64_t npq = (np + 3) >> 2;
  // workgroup g: pairs 4 (g / KSq) .. + 3 at K-split quad g % KSq (split
  // quads fastest: measured faster than pair quads fastest on 512x512 maps)
  const int64_t g = blockIdx.x;
  if (g >= npq * KSq) return;  // the whole workgroup is idle
  const int64_t pq = g / KSq, ksq = g - pq * KSq, p = 4 * pq + (wave >> 2);
  const int kq = wave & 3;
  auto setup = [&]() {
    build_lut(lds, a.ep);
    __syncthreads();
  };
  f32x16_t acc[3];
  int64_t lb = 0, rp = 0;
  if (p < np) {
    // pair p = row tiles 2 (p % prt) (+ 1) of the class's (p / prt)-th image
    const int64_t j = p / prt;
    rp = p - j * prt;
    const int64_t task = __builtin_amdgcn_readfirstlane(a.sched[kSchedList + j * rt + 2 * rp]);
    lb = task / rt;
    const uint32_t ring = (uint32_t)(size_t)(lds_void_t*)lds + ring_base(wave);
    cost_wave_pair(a, lb, 32 * rp, 4 * ksq + kq, 4 * KSq, lds, ring, acc, setup);
  } else {
    setup();
  }
  // sum the four splits of each pair: every wave has drained its loads, so
  // the table and the rings are free
  float* red = (float*)lds;
  constexpr int kAccFloats = 3 * 16 * 64;
  const int pp = wave >> 2;
  __syncthreads();
  if (p < np && kq >= 2) acc_to_lds(red + (2 * pp + kq - 2) * kAccFloats, acc, lane);
  __syncthreads();
  if (p < np && kq < 2) acc_add_lds(acc, red + (2 * pp + kq) * kAccFloats, lane);
  __syncthreads();
  if (p < np && kq == 1) acc_to_lds(red + pp * kAccFloats, acc, lane);
  __syncthreads();
  if (p >= np || kq != 0) return;
  acc_add_lds(acc, red + pp * kAccFloats, lane);

  // item ksq * np + p: [3][32 rows][32 slots]; rows of the second tile only
  // for a real pair, slots up to the ones column only (what the finalize reads)
  const int r = lane & 31, h = lane >> 5;
  const int G = __builtin_amdgcn_readfirstlane(a.ncols[lb % a.B]);
  const bool two = 2 * rp + 1 < rt;
  float* out = a.partials + a.plan.float_base[0] + (ksq * np + p) * kPairTile;
  if (r <= G) {
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = 8 * (v >> 2) + 4 * h + (v & 3);
        if (two || m < 16) out[(i * 32 + m) * 32 + r] = acc[i][v];
      }
  }
}

// ---- launch plan ---------------------------------------------------------------
// Resident waves of one cost kernel instance on the current device (cached).
template <int DT, int RT, int NT, int CNT, bool TAB>
static int occ_slots() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    int nb = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, cost_kernel<DT, RT, NT, CNT, TAB>, 64 * cost_waves(NT, TAB), 0) !=
            hipSuccess || nb < 1)
      nb = 1;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
      cus = 256;
    v = nb * cus * cost_waves(NT, TAB);
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

// The LDS-staged table kernel needs 16-byte aligned rows (HW % 8 == 0) whose
// per-tile element offsets fit 32 bits.
static bool dma_ok(const Dims& d) { return d.HW % 8 == 0 && d.HW >= 8 && d.HW * 16 < ((int64_t)1 << 31); }

// Resident waves of the LDS-staged table kernel on the current device (cached).
static int occ_slots_dma() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    int nb = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, cost_dma_kernel<2>, 64 * kDmaWaves, 0) !=
            hipSuccess || nb < 1)
      nb = 1;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
      cus = 256;
    v = nb * cus * (int)kDmaWaves;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

// Resident waves of the row-tile pair kernel on the current device (cached).
static int occ_slots_pair() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    int nb = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, cost_pair_kernel, 64 * kDmaWaves, 0) !=
            hipSuccess || nb < 1)
      nb = 1;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
      cus = 256;
    v = nb * cus * (int)kDmaWaves;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

// cnt: 0 label map, 1 u8 counts, 2 u16 counts
template <int DT, int RT, int NT>
static int occ_slots_for(int cnt, bool tab) {
  if (cnt == 1) return occ_slots<DT, RT, NT, 1, false>();
  if (cnt == 2) return occ_slots<DT, RT, NT, 2, false>();
  if (DT == ML_BF16 && tab) return occ_slots<DT, RT, NT, 0, DT == ML_BF16>();
  return occ_slots<DT, RT, NT, 0, false>();
}

static int cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v < 1) v = 256;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

// With three classes the narrower ones leave `side` CUs' worth of waves free:
// their launches may run beside the widest class's assignment (one
// workgroup per image on the forward's side stream).
template <int DT, int RT>
static void plan_slots(CostPlan& p, int cnt, bool tab, bool dma, int64_t side) {
  const int cus = cu_count();
  side = std::min<int64_t>(side, cus / 8);
  for (int ci = 0; ci < p.nclass; ++ci) {
    int v = 0;
    switch (ci) {
      case 0:
        v = p.pair0 ? occ_slots_pair()
            : DT == ML_BF16 && tab && cnt == 0 && dma ? occ_slots_dma()
                                                      : occ_slots_for<DT, RT, 2>(cnt, tab);
        break;
      case 1: v = occ_slots_for<DT, RT, 7>(cnt, tab); break;
      default: v = occ_slots_for<DT, RT, 16>(cnt, tab); break;
    }
    if (p.nclass == kClasses && ci < kClasses - 1) v -= (int)((int64_t)v * side / cus);
    p.slots[ci] = (int)std::min<int64_t>(std::max(v, 8), kCostSlots);
  }
}

CostPlan make_cost_plan(const Dims& d, int dtype, bool tab) {
  CostPlan p = bound_cost_plan(d);
  const int cnt = d.counts_mode ? d.cw : 0;
  p.pair0 = dtype == ML_BF16 && tab && d.pair_ok ? 1 : 0;
  // the wide classes' slot-sum form runs on label maps without the table
  for (int c = 0; c < kClasses; ++c) p.planes[c] = c > 0 && !d.counts_mode && !(dtype == ML_BF16 && tab) ? 4 : 3;
  const int64_t side = std::min<int64_t>(d.LB, kSideCUs);
  switch (dtype) {
    case ML_F32: plan_slots<ML_F32, 1>(p, cnt, false, false, side); break;
    case ML_BF16: plan_slots<ML_BF16, 1>(p, cnt, tab, dma_ok(d), side); break;
    case ML_F16: plan_slots<ML_F16, 1>(p, cnt, false, false, side); break;
  }
  return p;
}

template <int DT, int RT, int NT>
static int launch_one(const CostArgs& a, const Dims& d, bool tab, hipStream_t st) {
  constexpr int CI = kClassOf<NT>;
  if (NT == 2 && a.plan.pair0) {
    // the schedule's K-split was chosen for row-tile pairs
    if (DT != ML_BF16 || !tab || !d.pair_ok || d.rows != 16)
      return fail(ML_EINVAL, "internal: row-tile pair plan without the bf16 table path");
    // workgroups: ceil(np / 4) pair quads x KSq split quads, where np * 4 KSq
    // <= max(slots, np) unless KSq = 1 (then np <= L B ceil(rtiles / 2)), and
    // KSq <= ks_max / 4; surplus workgroups exit at once
    const int64_t np_max = d.LB * ((d.rtiles + 1) / 2);
    const int64_t wgs = ceil_div(a.plan.slots[CI], 16) + ceil_div(np_max, 4) + d.ks_max / 4 + 1;
    hipLaunchKernelGGL(cost_pair_kernel, dim3((unsigned)wgs), dim3(64 * kDmaWaves), 0, st, a);
    return check_launch("pair_cost");
  }
  if constexpr (DT == ML_BF16 && NT == 2) {
    if (tab && !d.counts_mode && dma_ok(d)) {
      const dim3 grid((unsigned)ceil_div(std::max<int64_t>(a.plan.slots[CI], a.plan.ntasks), kDmaWaves));
      hipLaunchKernelGGL((cost_dma_kernel<NT>), grid, dim3(64 * kDmaWaves), 0, st, a);
      return check_launch("pair_cost");
    }
  }
  const int WV = cost_waves(NT, DT == ML_BF16 && tab && !d.counts_mode);
  const dim3 grid((unsigned)ceil_div(std::max<int64_t>(a.plan.slots[CI], a.plan.ntasks), WV));
  if (d.counts_mode && d.cw == 2)
    hipLaunchKernelGGL((cost_kernel<DT, RT, NT, 2, false>), grid, dim3(64 * WV), 0, st, a);
  else if (d.counts_mode)
    hipLaunchKernelGGL((cost_kernel<DT, RT, NT, 1, false>), grid, dim3(64 * WV), 0, st, a);
  else if (DT == ML_BF16 && tab)
    hipLaunchKernelGGL((cost_kernel<DT, RT, NT, 0, DT == ML_BF16>), grid, dim3(64 * WV), 0, st, a);
  else
    hipLaunchKernelGGL((cost_kernel<DT, RT, NT, 0, false>), grid, dim3(64 * WV), 0, st, a);
  return check_launch("pair_cost");
}

// One launch per column-tile class up to the padded width; each image is
// processed by exactly one of them.
template <int DT, int RT>
static int launch_classes(const CostArgs& a, const Dims& d, bool tab, unsigned classes, hipStream_t st) {
  int rc = 0;
  if (classes & 1u) rc = launch_one<DT, RT, 2>(a, d, tab, st);
  if (!rc && a.plan.nclass > 1 && (classes & 2u)) rc = launch_one<DT, RT, 7>(a, d, tab, st);
  if (!rc && a.plan.nclass > 2 && (classes & 4u)) rc = launch_one<DT, RT, 16>(a, d, tab, st);
  return rc;
}

int cost_rt_for(int, int) { return 1; }

int launch_cost(const CostArgs& a, const Dims& d, int dtype, bool, hipStream_t st, unsigned classes,
                bool prof) {
  ProfScope ps_(prof ? "pair_cost" : nullptr, st);
  // bf16 with label maps and no unweighted row sums: table path
  const bool tab = dtype == ML_BF16 && !d.counts_mode && a.use_lut && a.rowsum == nullptr;
  switch (dtype) {
    case ML_F32: return launch_classes<ML_F32, 1>(a, d, false, classes, st);
    case ML_BF16: return launch_classes<ML_BF16, 1>(a, d, tab, classes, st);
    case ML_F16: return launch_classes<ML_F16, 1>(a, d, false, classes, st);
  }
  return fail(ML_EINVAL, "unsupported mask logits dtype");
}

}  // namespace ml
