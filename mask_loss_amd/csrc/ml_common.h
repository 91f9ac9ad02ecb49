// Shared device helpers and parameter blocks for the mask-cost / assignment /
// matched-loss kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mask_loss_hip.h"

namespace ml {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kEps = 1e-12f;
constexpr uint16_t kNoLabel = 0xFFFFu;

// ---------------------------------------------------------------------------
// element type helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t x) { return __uint_as_float(x << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t x) { return __uint_as_float(x & 0xFFFF0000u); }

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  f32x2_t f = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}
__device__ __forceinline__ float bf16_round(float a) {  // value after RNE to bf16
  return bf16_lo(pack_bf16x2(a, 0.f));
}

__device__ __forceinline__ float load_elem(const float* p, int64_t i) { return p[i]; }
__device__ __forceinline__ float load_elem(const uint16_t* p, int64_t i) {
  return __uint_as_float(((uint32_t)p[i]) << 16);
}
__device__ __forceinline__ float load_elem_f16(const uint16_t* p, int64_t i) {
  return (float)__builtin_bit_cast(_Float16, p[i]);
}

// ---------------------------------------------------------------------------
// packed 16-bit integer helpers (one-hot target operands); pk_min_u16 and
// pk_sub_sat_u16 take their second operand in a scalar register, so it must be
// wave-uniform (every caller passes a constant)
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t pk_min_u16(uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_pk_min_u16 %0, %1, %2" : "=v"(r) : "v"(a), "s"(b));
  return r;
}
__device__ __forceinline__ uint32_t pk_mul_lo_u16(uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_pk_mul_lo_u16 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ uint32_t pk_sub_sat_u16(uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_pk_sub_u16 %0, %1, %2 clamp" : "=v"(r) : "v"(a), "s"(b));
  return r;
}
__device__ __forceinline__ uint32_t pk_sub_u16(uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_pk_sub_u16 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// ---------------------------------------------------------------------------
// per-element loss terms
// ---------------------------------------------------------------------------
// Parameters of the per-logit terms (focal modulation, uncertainty weight).
struct ElemParams {
  float an, ap;       // focal alphas (1,1 when disabled)
  float gamma;        // focal gamma
  float ug, ug_min;   // uncertainty gamma and floor
  int gamma_mode;     // 0: gamma == 0, 1: gamma == 1, 2: gamma == 2, 3: general
  int ug_mode;        // 0: ug == 0 (w = 1), 1: ug == 1 (w = H), 2: general (w = H^ug)
};

__host__ inline ElemParams make_elem_params(float gamma, float alpha, float ug, float ug_min) {
  ElemParams e;
  e.ap = alpha >= 0.f ? alpha : 1.f;
  e.an = alpha >= 0.f ? 1.f - alpha : 1.f;
  e.gamma = gamma;
  e.gamma_mode = gamma > 0.f ? (gamma == 1.f ? 1 : (gamma == 2.f ? 2 : 3)) : 0;
  e.ug = ug;
  e.ug_min = ug_min;
  e.ug_mode = ug != 0.f ? (ug == 1.f ? 1 : 2) : 0;
  return e;
}

// Sigmoid-BCE building blocks of one logit z, all without cancellation:
//   p = sigmoid(z), q1 = 1 - p, cp = softplus(-z) = -log p, cn = softplus(z) = -log(1-p)
struct Sig {
  float p, q1, cp, cn;
};
__device__ __forceinline__ Sig sig_terms(float z) {
  const float e = __builtin_amdgcn_exp2f(-fabsf(z) * kLog2e);  // exp(-|z|) in (0,1]
  const float d = 1.0f + e;
  const float r = __builtin_amdgcn_rcpf(d);
  const float l1 = __builtin_amdgcn_logf(d) * kLn2;  // log1p(exp(-|z|))
  const float er = e * r;
  const bool pos = z >= 0.f;
  Sig s;
  s.p = pos ? r : er;
  s.q1 = pos ? er : r;
  s.cn = l1 + fmaxf(z, 0.f);
  s.cp = l1 + fmaxf(-z, 0.f);
  return s;
}

// Clamped entropy weight w = clamp(H(p)^ug, ug_min, 1), H in bits.
__device__ __forceinline__ float unc_weight(const Sig& s, const ElemParams& ep) {
  float w = 1.0f;
  if (ep.ug_mode != 0) {
    float h = fmaf(s.p, s.cp, s.q1 * s.cn) * kLog2e;  // -(p ln p + (1-p) ln(1-p)) / ln 2
    if (ep.ug_mode == 2) h = __builtin_amdgcn_exp2f(ep.ug * __builtin_amdgcn_logf(h));
    w = h;
  }
  return __builtin_amdgcn_fmed3f(w, ep.ug_min, 1.0f);
}

// Focal modulators mn = p^gamma, mp = (1-p)^gamma (ln p = -cp, ln(1-p) = -cn).
__device__ __forceinline__ void focal_mods(const Sig& s, const ElemParams& ep, float& mn, float& mp) {
  if (ep.gamma_mode == 0) {
    mn = 1.f;
    mp = 1.f;
  } else if (ep.gamma_mode == 1) {
    mn = s.p;
    mp = s.q1;
  } else if (ep.gamma_mode == 2) {
    mn = s.p * s.p;
    mp = s.q1 * s.q1;
  } else {
    mn = __builtin_amdgcn_exp2f(-ep.gamma * s.cp * kLog2e);
    mp = __builtin_amdgcn_exp2f(-ep.gamma * s.cn * kLog2e);
  }
}

// The same terms with the modes fixed at compile time where EM = 1: no
// focal modulation (gamma = 0) and the uncertainty weight H(p)^1, the
// operator's default arguments.  The arithmetic is that of unc_weight /
// focal_mods for those modes, without a branch on the modes per logit;
// EM = 0 is the general form.  Callers pick EM once per group of logits
// (default_modes).
__device__ __forceinline__ bool default_modes(const ElemParams& ep) {
  return ep.gamma_mode == 0 && ep.ug_mode == 1;
}
template <int EM>
__device__ __forceinline__ float unc_weight_m(const Sig& s, const ElemParams& ep) {
  if constexpr (EM == 1) {
    const float h = fmaf(s.p, s.cp, s.q1 * s.cn) * kLog2e;
    return __builtin_amdgcn_fmed3f(h, ep.ug_min, 1.0f);
  } else {
    return unc_weight(s, ep);
  }
}
template <int EM>
__device__ __forceinline__ void focal_mods_m(const Sig& s, const ElemParams& ep, float& mn, float& mp) {
  if constexpr (EM == 1) {
    mn = 1.f;
    mp = 1.f;
  } else {
    focal_mods(s, ep, mn, mp);
  }
}

// ---------------------------------------------------------------------------
// wave reductions (wave64)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace ml
