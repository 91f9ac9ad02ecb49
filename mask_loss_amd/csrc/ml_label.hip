// Standalone pairwise label cost (L,B,Q,GT_out): sigmoid one-hot BCE
// (src/cuda/pw_sigmoid_label_loss.cu:16-106) or softmax CE
// (src/cuda/pw_softmax_label_loss.cu:12-103).  One wave per (l,b,q) row.
#include "ml_internal.h"

namespace ml {

struct LabelArgs {
  const void* z;
  int dt;
  const int64_t* tg;
  float* out;
  int64_t L, B, Q, C, GT_total, GT_out, bg;
  float scale;
  ElemParams ep;
  int use_softmax;
};

__device__ __forceinline__ float lab_in(const void* p, int dt, int64_t i) {
  if (dt == ML_F32) return ((const float*)p)[i];
  const uint16_t h = ((const uint16_t*)p)[i];
  if (dt == ML_BF16) return __uint_as_float(((uint32_t)h) << 16);
  return (float)__builtin_bit_cast(_Float16, h);
}

__global__ __launch_bounds__(256) void label_cost_kernel(LabelArgs a) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= a.L * a.B * a.Q) return;
  const int64_t b = (row / a.Q) % a.B;
  const int64_t zb = row * a.C;
  float rowv;
  if (a.use_softmax) {
    float m = -INFINITY;
    for (int64_t c = lane; c < a.C; c += 64) m = fmaxf(m, lab_in(a.z, a.dt, zb + c));
    m = wave_max(m);
    float se = 0.f;
    for (int64_t c = lane; c < a.C; c += 64) se += __expf(lab_in(a.z, a.dt, zb + c) - m);
    se = wave_sum(se);
    rowv = __logf(fmaxf(se, 1e-20f)) + m;
  } else {
    float base = 0.f;
    for (int64_t c = lane; c < a.C; c += 64) {
      const Sig s = sig_terms(lab_in(a.z, a.dt, zb + c));
      float mn, mp;
      focal_mods(s, a.ep, mn, mp);
      base += a.ep.an * mn * s.cn;
    }
    rowv = wave_sum(base);
  }
  for (int64_t k = lane; k < a.GT_out; k += 64) {
    const int64_t act = k + (k >= a.bg ? 1 : 0);
    const int64_t y = a.tg[b * a.GT_total + act];
    float v;
    if (y < 0 || y >= a.C) {
      v = INFINITY;
    } else {
      const float zy = lab_in(a.z, a.dt, zb + y);
      if (a.use_softmax) {
        v = (rowv - zy) * a.scale;
      } else {
        const Sig s = sig_terms(zy);
        float mn, mp;
        focal_mods(s, a.ep, mn, mp);
        const float delta = a.ep.ap * mp * s.cp - a.ep.an * mn * s.cn;
        v = (rowv + delta) * (1.f / (float)a.C) * a.scale;
      }
    }
    a.out[row * a.GT_out + k] = v;
  }
}

int launch_label_cost(const void* cls_logits, int cls_dtype, const int64_t* cls_targets,
                      int64_t L, int64_t B, int64_t Q, int64_t C, int64_t GT_total,
                      int64_t GT_out, int64_t bg, float scale, const ElemParams& ep,
                      int use_softmax, float* out, hipStream_t st) {
  const int64_t rows = L * B * Q;
  if (rows == 0 || GT_out == 0) return ML_OK;
  LabelArgs a{cls_logits, cls_dtype, cls_targets, out, L, B, Q, C, GT_total, GT_out, bg,
              scale, ep, use_softmax};
  hipLaunchKernelGGL(label_cost_kernel, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, st, a);
  return check_launch("label_cost");
}

}  // namespace ml
