// Per-element optimizer arithmetic shared by the streaming optimizer kernel and the fused
// dW-GEMM epilogue: binary32 operations in the order of TrainingParameter.stageUpdate32
// (TrainingParameter.java:622-672) and stageAdaptiveElement32 (:433-525), every intermediate
// checked finite.
#pragma once
#include "common.h"
#include "kernels.h"

namespace shk {

struct Coeffs {
  float c1, c2, decay_factor;
  bool ok;
};

template <typename P>
__device__ __forceinline__ Coeffs adam_coeffs(const P& p, int64_t step) {
  Coeffs k;
  k.c1 = 1.0f - (float)pow((double)p.beta1, (double)step);
  k.c2 = 1.0f - (float)pow((double)p.beta2, (double)step);
  k.ok = is_finite(k.c1) && k.c1 > 0.0f && is_finite(k.c2) && k.c2 > 0.0f;
  k.decay_factor = 1.0f;
  if (p.kind == 2) {
    const float scale = p.lr * p.weight_decay;
    k.ok = k.ok && is_finite(scale);
    k.decay_factor = k.decay_factor - scale;
    k.ok = k.ok && is_finite(k.decay_factor);
  }
  return k;
}

// Finiteness checks without lane-mask arithmetic: chk = fmaf(x, 0, chk) turns NaN as soon as one
// checked value is +-inf or NaN and otherwise stays +0, so one comparison after a whole block of
// elements (chk == 0) says whether every intermediate was finite. A comparison per check would
// give a lane mask combined by scalar instructions, each waiting for the vector compare before
// it; this is one vector FMA per check.
__device__ __forceinline__ void check_finite(float x, float& chk) { chk = fmaf(x, 0.0f, chk); }
__device__ __forceinline__ void check_positive(float x, float& chk) {
  chk = x > 0.0f ? chk : __int_as_float(0x7fc00000);
}

// One SGD element; non-finite intermediates turn chk NaN.
template <typename P>
__device__ __forceinline__ void sgd_element(const P& p, bool first, float pv, float g, float mv,
                                            float& pc, float& mc, float& chk) {
  check_finite(pv, chk);
  const float decay_term = p.weight_decay * pv;
  check_finite(decay_term, chk);
  const float adjusted = g + decay_term;
  check_finite(adjusted, chk);
  float selected = adjusted;
  mc = mv;
  if (p.momentum != 0.0f) {
    float um;
    if (first) {
      um = adjusted;
    } else {
      const float mt = p.momentum * mv;
      check_finite(mt, chk);
      const float dg = (1.0f - p.dampening) * adjusted;
      check_finite(dg, chk);
      um = mt + dg;
    }
    check_finite(um, chk);
    mc = um;
    if (p.nesterov) {
      const float look = p.momentum * um;
      check_finite(look, chk);
      selected = adjusted + look;
      check_finite(selected, chk);
    } else {
      selected = um;
    }
  } else if (p.has_momentum_slot) {
    mc = 0.0f;
  }
  const float scaled = p.lr * selected;
  check_finite(scaled, chk);
  pc = pv - scaled;
  check_finite(pc, chk);
}

// One Adam/AdamW element; non-finite intermediates and a denominator that is not positive turn
// chk NaN.
template <typename P>
__device__ __forceinline__ void adam_element(const P& p, const Coeffs& k, float pv, float g0,
                                             float mv, float vv, float& pc, float& mc, float& vc,
                                             float& chk) {
  check_finite(pv, chk);
  float gradient, base;
  if (p.kind == 2) {
    base = pv * k.decay_factor;
    check_finite(base, chk);
    gradient = g0;
  } else {
    const float decay_term = p.weight_decay * pv;
    check_finite(decay_term, chk);
    gradient = g0 + decay_term;
    check_finite(gradient, chk);
    base = pv;
  }
  const float first_term = p.beta1 * mv;
  check_finite(first_term, chk);
  const float first_grad = (1.0f - p.beta1) * gradient;
  check_finite(first_grad, chk);
  const float first = first_term + first_grad;
  check_finite(first, chk);
  const float squared = gradient * gradient;
  check_finite(squared, chk);
  const float second_term = p.beta2 * vv;
  check_finite(second_term, chk);
  const float second_grad = (1.0f - p.beta2) * squared;
  check_finite(second_grad, chk);
  const float second = second_term + second_grad;
  check_finite(second, chk);
  const float cf = first / k.c1;
  const float cs = second / k.c2;
  check_finite(cf, chk);
  check_finite(cs, chk);
  const float root = (float)sqrt((double)cs);
  check_finite(root, chk);
  const float denom = root + p.eps;
  check_finite(denom, chk);
  check_positive(denom, chk);
  const float numer = p.lr * cf;
  check_finite(numer, chk);
  const float update = numer / denom;
  check_finite(update, chk);
  pc = base - update;
  check_finite(pc, chk);
  mc = first;
  vc = second;
}


}  // namespace shk
