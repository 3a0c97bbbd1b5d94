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

// One SGD element. Returns false if any intermediate is not finite.
template <typename P>
__device__ __forceinline__ bool sgd_element(const P& p, bool first, float pv, float g,
                                            float mv, float& pc, float& mc) {
  bool ok = is_finite(pv);
  const float decay_term = p.weight_decay * pv;
  ok &= is_finite(decay_term);
  const float adjusted = g + decay_term;
  ok &= is_finite(adjusted);
  float selected = adjusted;
  mc = mv;
  if (p.momentum != 0.0f) {
    float um;
    if (first) {
      um = adjusted;
    } else {
      const float mt = p.momentum * mv;
      ok &= is_finite(mt);
      const float dg = (1.0f - p.dampening) * adjusted;
      ok &= is_finite(dg);
      um = mt + dg;
    }
    ok &= is_finite(um);
    mc = um;
    if (p.nesterov) {
      const float look = p.momentum * um;
      ok &= is_finite(look);
      selected = adjusted + look;
      ok &= is_finite(selected);
    } else {
      selected = um;
    }
  } else if (p.has_momentum_slot) {
    mc = 0.0f;
  }
  const float scaled = p.lr * selected;
  ok &= is_finite(scaled);
  pc = pv - scaled;
  ok &= is_finite(pc);
  return ok;
}

// One Adam/AdamW element.
template <typename P>
__device__ __forceinline__ bool adam_element(const P& p, const Coeffs& k, float pv,
                                             float g0, float mv, float vv, float& pc, float& mc,
                                             float& vc) {
  bool ok = is_finite(pv);
  float gradient, base;
  if (p.kind == 2) {
    base = pv * k.decay_factor;
    ok &= is_finite(base);
    gradient = g0;
  } else {
    const float decay_term = p.weight_decay * pv;
    ok &= is_finite(decay_term);
    gradient = g0 + decay_term;
    ok &= is_finite(gradient);
    base = pv;
  }
  const float first_term = p.beta1 * mv;
  ok &= is_finite(first_term);
  const float first_grad = (1.0f - p.beta1) * gradient;
  ok &= is_finite(first_grad);
  const float first = first_term + first_grad;
  ok &= is_finite(first);
  const float squared = gradient * gradient;
  ok &= is_finite(squared);
  const float second_term = p.beta2 * vv;
  ok &= is_finite(second_term);
  const float second_grad = (1.0f - p.beta2) * squared;
  ok &= is_finite(second_grad);
  const float second = second_term + second_grad;
  ok &= is_finite(second);
  const float cf = first / k.c1;
  const float cs = second / k.c2;
  ok &= is_finite(cf) && is_finite(cs);
  const float root = (float)sqrt((double)cs);
  ok &= is_finite(root);
  const float denom = root + p.eps;
  ok &= is_finite(denom) && denom > 0.0f;
  const float numer = p.lr * cf;
  ok &= is_finite(numer);
  const float update = numer / denom;
  ok &= is_finite(update);
  pc = base - update;
  ok &= is_finite(pc);
  mc = first;
  vc = second;
  return ok;
}


}  // namespace shk
