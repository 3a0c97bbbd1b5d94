/*
 * CPU restatement of the reference's default CPU algorithms for the fp32 MLP training path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg load this library, as the checker or the timed CPU baseline; the product path
 * (synaptik_amd) never calls it.
 *
 * Compiled with -ffp-contract=off and without -ffast-math: every binary32 operation below is
 * one IEEE-754 rounded operation in the order the reference performs it. Each function cites
 * the reference file it restates. Transcendentals use glibc's correctly-rounded-in-practice
 * binary64 exp/log/tanh where the reference calls java.lang.StrictMath (fdlibm); the two agree
 * to within one binary64 ulp, which almost never changes the binary32 result (documented as
 * the unpinned part of the restatement).
 */
#include "synaptik_oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------------------------
 * MATMUL: CpuMatmulReferenceKernel.evaluate (modules/backend/cpu/src/main/java/io/github/
 * pho001/synaptik/backend/cpu/internal/reference/CpuMatmulReferenceKernel.java:34-119),
 * FLOAT32 branch with the no-FMA numerical form: every output starts at +0.0f and adds
 * x*y (two roundings) over increasing k exactly once; K == 1 is the single product; K == 0
 * keeps +0.0f. The loop is ordered m, k, n so that the independent per-n chains vectorize
 * without changing any element's operation order.
 * element (m,k) of A: trans_a ? A[k*lda + m] : A[m*lda + k]
 * element (k,n) of B: trans_b ? B[n*ldb + k] : B[k*ldb + n]
 * ------------------------------------------------------------------------------------------ */
void shko_matmul_f32(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K,
                     int64_t lda, int64_t ldb, int64_t ldc, int trans_a, int trans_b) {
  const float* Bn = B;
  float* Bt = NULL;
  if (trans_b && K > 0 && N > 0) {
    /* materialize B as [K,N] (the OpenBLAS route copies transposed operands the same way) */
    Bt = (float*)malloc(sizeof(float) * (size_t)K * (size_t)N);
    for (int64_t k = 0; k < K; ++k)
      for (int64_t n = 0; n < N; ++n) Bt[k * N + n] = B[n * ldb + k];
    Bn = Bt;
    ldb = N;
  }
  for (int64_t m = 0; m < M; ++m) {
    float* c = C + m * ldc;
    if (K == 1) {
      const float a = trans_a ? A[m] : A[m * lda];
      for (int64_t n = 0; n < N; ++n) c[n] = a * Bn[n];
      continue;
    }
    for (int64_t n = 0; n < N; ++n) c[n] = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      const float a = trans_a ? A[k * lda + m] : A[m * lda + k];
      const float* b = Bn + k * ldb;
      for (int64_t n = 0; n < N; ++n) {
        const float prod = a * b[n];
        c[n] = c[n] + prod;
      }
    }
  }
  free(Bt);
}

/* ------------------------------------------------------------------------------------------
 * Exact binary32 summation with one final round-to-nearest-even
 * (CpuExactSumEmitter.java:4-12: fixed-width limb accumulation rounded once;
 *  CpuAggregateEmitter.java:18-20: SUM/MEAN/SUM_TO_SHAPE use it).
 * Every finite binary32 is an integer multiple of 2^-149 below 2^128, so a 320-bit two's
 * complement fixed-point accumulator (10 x 32-bit limbs, carry-saved in int64) is exact.
 * ------------------------------------------------------------------------------------------ */
#define SA_LIMBS 10
typedef struct {
  int64_t limb[SA_LIMBS];
  int64_t adds;
  int nan, pinf, ninf;
} superacc;

static void sa_init(superacc* s) { memset(s, 0, sizeof *s); }

static void sa_normalize(superacc* s) {
  int64_t carry = 0;
  for (int i = 0; i < SA_LIMBS; ++i) {
    int64_t v = s->limb[i] + carry;
    int64_t lo = v & 0xffffffffll;
    carry = (v - lo) / 4294967296ll; /* exact: v - lo is a multiple of 2^32 */
    s->limb[i] = lo;
  }
  /* the top carry holds the sign (the range guarantees no overflow) */
  s->limb[SA_LIMBS - 1] += carry * 4294967296ll;
  s->adds = 0;
}

static void sa_add(superacc* s, float x) {
  if (x != x) { s->nan = 1; return; }
  if (isinf(x)) { if (x > 0) s->pinf = 1; else s->ninf = 1; return; }
  if (x == 0.0f) return;
  uint32_t bits;
  memcpy(&bits, &x, 4);
  const int neg = bits >> 31;
  const int be = (bits >> 23) & 0xff;
  uint64_t mant = bits & 0x7fffff;
  int e; /* value = mant * 2^(e - 149) */
  if (be == 0) e = 0;
  else { mant |= 0x800000; e = be - 1; }
  const int limb = e / 32, sh = e % 32;
  const uint64_t v = mant << sh; /* < 2^56 */
  const int64_t lo = (int64_t)(v & 0xffffffffull), hi = (int64_t)(v >> 32);
  if (neg) { s->limb[limb] -= lo; s->limb[limb + 1] -= hi; }
  else { s->limb[limb] += lo; s->limb[limb + 1] += hi; }
  if (++s->adds >= (1ll << 29)) sa_normalize(s);
}

/* Rounds the magnitude Q * 2^exp2 (Q given as little-endian uint32 limbs) plus a sticky
 * indication of a nonzero remainder below Q's last bit to binary32, RNE, with subnormals. */
static float round_to_float(const uint32_t* q, int nlimbs, int exp2, int sticky, int neg) {
  int top = -1;
  for (int i = nlimbs - 1; i >= 0; --i)
    if (q[i]) { top = i; break; }
  if (top < 0) return neg ? -0.0f : 0.0f; /* only reached for an exact zero */
  int nb = top * 32 + (32 - __builtin_clz(q[top]));
  /* lowest representable bit position (relative to Q's bit 0) for the result */
  /* value exponent of the leading bit: nb - 1 + exp2 */
  int lead = nb - 1 + exp2;
  int keep_bits = 24;
  if (lead < -126) keep_bits = 24 - (-126 - lead); /* subnormal: fewer significant bits */
  if (keep_bits < 0) keep_bits = 0;
  int shift = nb - keep_bits; /* bits dropped */
  uint64_t keep = 0;
  int half = 0, low = sticky;
  if (shift <= 0) {
    for (int b = nb - 1; b >= 0; --b) keep = (keep << 1) | ((q[b / 32] >> (b % 32)) & 1u);
    keep <<= -shift;
    shift = shift < 0 ? shift : 0;
  } else {
    for (int b = nb - 1; b >= shift; --b) keep = (keep << 1) | ((q[b / 32] >> (b % 32)) & 1u);
    half = (q[(shift - 1) / 32] >> ((shift - 1) % 32)) & 1u;
    for (int b = shift - 2; b >= 0 && !low; --b) low |= (q[b / 32] >> (b % 32)) & 1u;
    if (half && (low || (keep & 1u))) keep++;
  }
  /* value = keep * 2^(shift + exp2) */
  double r = ldexp((double)keep, shift + exp2);
  float f = (float)r; /* exact unless it overflows to infinity */
  if (r > 3.4028234663852886e38) f = INFINITY;
  return neg ? -f : f;
}

static float sa_result(superacc* s, int64_t divisor) {
  if (s->nan || (s->pinf && s->ninf)) return NAN;
  if (s->pinf) return INFINITY;
  if (s->ninf) return -INFINITY;
  sa_normalize(s);
  int neg = s->limb[SA_LIMBS - 1] < 0;
  uint32_t mag[SA_LIMBS + 2];
  memset(mag, 0, sizeof mag);
  /* two's complement magnitude */
  uint64_t carry = neg ? 1 : 0;
  for (int i = 0; i < SA_LIMBS; ++i) {
    uint32_t w = (uint32_t)(s->limb[i] & 0xffffffffll);
    if (neg) {
      uint64_t v = (uint64_t)(uint32_t)~w + carry;
      mag[i] = (uint32_t)v;
      carry = v >> 32;
    } else {
      mag[i] = w;
    }
  }
  int any = 0;
  for (int i = 0; i < SA_LIMBS; ++i) any |= mag[i] != 0;
  if (!any) return 0.0f; /* exact zero sums to +0.0 */
  if (divisor == 1) return round_to_float(mag, SA_LIMBS, -149, 0, neg);
  /* exact rational quotient: shift left by 64 bits, long-divide by the divisor */
  uint32_t num[SA_LIMBS + 2];
  num[0] = 0; num[1] = 0;
  for (int i = 0; i < SA_LIMBS; ++i) num[i + 2] = mag[i];
  uint32_t quo[SA_LIMBS + 2];
  unsigned __int128 rem = 0;
  for (int i = SA_LIMBS + 1; i >= 0; --i) {
    unsigned __int128 cur = (rem << 32) | num[i];
    quo[i] = (uint32_t)(cur / (uint64_t)divisor);
    rem = cur % (uint64_t)divisor;
  }
  return round_to_float(quo, SA_LIMBS + 2, -149 - 64, rem != 0, neg);
}

float shko_exact_sum(const float* x, int64_t n, int64_t stride) {
  superacc s;
  sa_init(&s);
  for (int64_t i = 0; i < n; ++i) sa_add(&s, x[i * stride]);
  return sa_result(&s, 1);
}

float shko_exact_mean(const float* x, int64_t n, int64_t stride) {
  if (n == 0) return NAN;
  superacc s;
  sa_init(&s);
  for (int64_t i = 0; i < n; ++i) sa_add(&s, x[i * stride]);
  return sa_result(&s, n);
}

/* SUM_TO_SHAPE over rows: out[c] = exact sum_r X[r, c] (ElementwiseGradientRules.java:99-105,
 * TensorSumToShapeExpressions.java:173). */
void shko_colsum(const float* X, float* out, int64_t R, int64_t N, int64_t ldx) {
  for (int64_t c = 0; c < N; ++c) out[c] = shko_exact_sum(X + c, R, ldx);
}

/* Exactly rounded value / count (CpuLossReferenceKernel.exactCountQuotient:221-225). */
float shko_exact_quotient(float value, int64_t count) {
  if (!isfinite(value) || value == 0.0f || count == 0) return value / (float)count;
  superacc s;
  sa_init(&s);
  sa_add(&s, value);
  return sa_result(&s, count);
}

/* ------------------------------------------------------------------------------------------
 * Activations: CpuScalarReferenceKernel.java:1213-1217 (two-branch sigmoid),
 * :1736-1737 (RELU = Math.max(x, +0.0), TANH = StrictMath.tanh), evaluated in binary64 and
 * narrowed once. Gradients: ElementwiseGradientRules.java:205-210.
 * act: 0 none, 1 relu, 2 tanh, 3 sigmoid
 * ------------------------------------------------------------------------------------------ */
static float act_fwd(int act, float x) {
  switch (act) {
    case 1: return (x > 0.0f || x != x) ? x : 0.0f;
    case 2: return (float)tanh((double)x);
    case 3: {
      double v = (double)x;
      if (v >= 0.0) return (float)(1.0 / (1.0 + exp(-v)));
      double e = exp(v);
      return (float)(e / (1.0 + e));
    }
    default: return x;
  }
}

static float act_bwd(int act, float g, float y) {
  switch (act) {
    case 1: return y > 0.0f ? g : 0.0f;
    case 2: { float yy = y * y; float d = 1.0f - yy; return g * d; }
    case 3: { float gy = g * y; float d = 1.0f - y; return gy * d; }
    default: return g;
  }
}

void shko_activation(int act, const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = act_fwd(act, x[i]);
}

void shko_activation_grad(int act, const float* g, const float* y, float* dx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dx[i] = act_bwd(act, g[i], y[i]);
}

/* Linear forward as the compiler builds it: input.matmul(weight.transpose()).add(bias)
 * (TensorLinearExpressions.java:97-146), then the activation. W is [out,in]. */
void shko_linear_forward(const float* X, const float* W, const float* b, float* Y, int64_t B,
                         int64_t in, int64_t out, int act) {
  shko_matmul_f32(X, W, Y, B, out, in, in, in, out, 0, 1);
  for (int64_t r = 0; r < B; ++r)
    for (int64_t c = 0; c < out; ++c) {
      float z = Y[r * out + c];
      if (b) z = z + b[c];
      Y[r * out + c] = act_fwd(act, z);
    }
}

/* ------------------------------------------------------------------------------------------
 * SOFTMAX / LOG_SOFTMAX rows: CpuSoftmaxReferenceKernel.evaluateFloat
 * (CpuSoftmaxReferenceKernel.java:104-146), including the +inf-maximum class rule, the
 * unshifted literal path for rows with -inf, and the Kahan-compensated binary32 sum.
 * ------------------------------------------------------------------------------------------ */
static float java_max(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  if (a == 0.0f && b == 0.0f) return signbit(a) ? b : a;
  return a > b ? a : b;
}

/* Floating MAX reduction (AggregateReductionKind.java:128-137): a left fold from the empty
 * domain's -infinity with java_max above -- a NaN operand makes the result NaN (its payload is
 * unspecified, foundational-modules.md:228), +0 is selected over -0, and values are compared
 * as stored (the comparisons are exact, subnormals are never flushed). */
float shko_max(const float* x, int64_t n, int64_t stride) {
  float m = -INFINITY;
  for (int64_t i = 0; i < n; ++i) m = java_max(m, x[i * stride]);
  return m;
}

void shko_softmax_rows(const float* X, float* Y, int64_t R, int64_t C, int log_softmax) {
  for (int64_t r = 0; r < R; ++r) {
    const float* x = X + r * C;
    float* y = Y + r * C;
    float maximum = -INFINITY;
    int unshifted = 0;
    for (int64_t c = 0; c < C; ++c) {
      maximum = java_max(maximum, x[c]);
      unshifted |= x[c] == -INFINITY;
    }
    if (maximum == INFINITY) {
      for (int64_t c = 0; c < C; ++c)
        y[c] = x[c] == INFINITY ? NAN : (log_softmax ? -INFINITY : 0.0f);
      continue;
    }
    if (unshifted && maximum == maximum) maximum = 0.0f;
    float sum = 0.0f, comp = 0.0f;
    for (int64_t c = 0; c < C; ++c) {
      float addend = (float)exp((double)(x[c] - maximum));
      if (unshifted) sum += addend;
      else {
        float adjusted = addend - comp, temporary = sum + adjusted;
        comp = (temporary - sum) - adjusted;
        sum = temporary;
      }
    }
    float logarithm = log_softmax ? (float)log((double)sum) : 0.0f;
    for (int64_t c = 0; c < C; ++c) {
      float shift = x[c] - maximum;
      y[c] = log_softmax ? shift - logarithm : (float)exp((double)shift) / sum;
    }
  }
}

/* LOG_SUM_EXP rows (CpuLogSumExpEmitter.java:4-9: two passes, shifted EXP, compensated sum,
 * LOG finishing), FLOAT32 sites: maximum, Kahan sum of (float)exp(x - maximum), then
 * maximum + (float)log(sum). A +inf or NaN maximum is returned as is; an all -inf row gives
 * -inf. */
void shko_logsumexp_rows(const float* X, float* out, int64_t R, int64_t C) {
  for (int64_t r = 0; r < R; ++r) {
    const float* x = X + r * C;
    float maximum = -INFINITY;
    for (int64_t c = 0; c < C; ++c) maximum = java_max(maximum, x[c]);
    if (maximum != maximum || maximum == INFINITY || maximum == -INFINITY) {
      out[r] = maximum;
      continue;
    }
    float sum = 0.0f, comp = 0.0f;
    for (int64_t c = 0; c < C; ++c) {
      float addend = (float)exp((double)(x[c] - maximum));
      float adjusted = addend - comp, temporary = sum + adjusted;
      comp = (temporary - sum) - adjusted;
      sum = temporary;
    }
    out[r] = maximum + (float)log((double)sum);
  }
}

/* SOFTMAX gradient y (.) (g - SUM(g (.) y)) (ReductionGradientRules.java:84-90); the row sum
 * is the exact SUM. */
void shko_softmax_grad_rows(const float* Y, const float* G, float* DX, int64_t R, int64_t C) {
  float* prod = (float*)malloc(sizeof(float) * (size_t)(C > 0 ? C : 1));
  for (int64_t r = 0; r < R; ++r) {
    const float* y = Y + r * C;
    const float* g = G + r * C;
    for (int64_t c = 0; c < C; ++c) prod[c] = g[c] * y[c];
    const float s = shko_exact_sum(prod, C, 1);
    for (int64_t c = 0; c < C; ++c) {
      float d = g[c] - s;
      DX[r * C + c] = y[c] * d;
    }
  }
  free(prod);
}

/* LOG_SUM_EXP gradient g_r * exp(x - lse_r) (ReductionGradientRules.java:213-224). */
void shko_logsumexp_grad_rows(const float* X, const float* lse, const float* g, float* DX,
                              int64_t R, int64_t C) {
  for (int64_t r = 0; r < R; ++r)
    for (int64_t c = 0; c < C; ++c) {
      float shifted = X[r * C + c] - lse[r];
      DX[r * C + c] = g[r] * (float)exp((double)shifted);
    }
}

/* ------------------------------------------------------------------------------------------
 * Losses: CpuLossReferenceKernel (reference/CpuLossReferenceKernel.java).
 * ------------------------------------------------------------------------------------------ */
/* meanSquaredError(float[], float[], MEAN) :67-87 — sequential binary32 sum, exact quotient. */
float shko_mse_mean(const float* p, const float* t, int64_t n) {
  float sum = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    float d = p[i] - t[i];
    float sq = d * d;
    sum += sq;
  }
  return shko_exact_quotient(sum, n);
}

/* MSE MEAN as the Model contract states it (foundational-modules.md:343: one subtraction and
 * delta*delta per position, "then its exact reduction and optional divisor"): the binary32
 * squares summed exactly and divided by n with one rounding. The reference's CPU kernels sum
 * the squares sequentially in binary32 instead (shko_mse_mean above; the generated kernel
 * CpuLossEmitter.emitContiguousMseInt:879-935 does the same), which drifts from this once the
 * running sum's ulp approaches the squares. */
float shko_mse_mean_exact(const float* p, const float* t, int64_t n) {
  if (n == 0) return NAN;
  superacc s;
  sa_init(&s);
  for (int64_t i = 0; i < n; ++i) {
    float d = p[i] - t[i];
    float sq = d * d;
    sa_add(&s, sq);
  }
  return sa_result(&s, n);
}

/* meanSquaredError(float[], float[], SUM): the sequential binary32 sum itself. */
float shko_mse_sum(const float* p, const float* t, int64_t n) {
  float sum = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    float d = p[i] - t[i];
    float sq = d * d;
    sum += sq;
  }
  return sum;
}

/* MSE MEAN gradient ((p - t) * 2) * (g / count) (LossGradientRules.java:77-97 with restore()
 * dividing the expanded cotangent by the exact element count). */
void shko_mse_grad(const float* p, const float* t, float* grad, int64_t n, float g, int sum) {
  const float gn = sum ? g : g / (float)n;
  for (int64_t i = 0; i < n; ++i) {
    float d = p[i] - t[i];
    float twice = d * 2.0f;
    grad[i] = twice * gn;
  }
}

static float ce_logsumexp(const float* v, int64_t C) {
  float maximum = -INFINITY;
  for (int64_t c = 0; c < C; ++c)
    if (v[c] > maximum) maximum = v[c];
  float sum = 0.0f;
  for (int64_t c = 0; c < C; ++c) {
    float shifted = v[c] - maximum;
    sum += (float)exp((double)shifted);
  }
  return maximum + (float)log((double)sum);
}

/* indexCategoricalCrossEntropy(float[], long[], ..., MEAN) :196-218,261-288.
 * Returns 0 on success, 1 if a non-ignored target lies outside [0, C) (the reference throws
 * IllegalArgumentException). */
int shko_index_ce_mean(const float* logits, const int64_t* target, int64_t R, int64_t C,
                       int has_ignore, int64_t ignore, float* loss) {
  float sum = 0.0f;
  int64_t count = 0;
  for (int64_t r = 0; r < R; ++r) {
    int64_t t = target[r];
    if (has_ignore && t == ignore) continue;
    if (t < 0 || t >= C) return 1;
    sum += ce_logsumexp(logits + r * C, C) - logits[r * C + t];
    count++;
  }
  *loss = sum / (float)count;
  return 0;
}

/* Index CE gradient (LossGradientRules.java:172-240):
 * (exp(l - max) / SUM(exp(l - max)) - onehot(clamp(t))) * (g / count), ignored rows 0. */
void shko_index_ce_grad(const float* logits, const int64_t* target, float* grad, int64_t R,
                        int64_t C, int has_ignore, int64_t ignore, float g) {
  int64_t count = 0;
  for (int64_t r = 0; r < R; ++r) count += !(has_ignore && target[r] == ignore);
  const float scale = g / (float)count;
  float* e = (float*)malloc(sizeof(float) * (size_t)(C > 0 ? C : 1));
  for (int64_t r = 0; r < R; ++r) {
    const float* l = logits + r * C;
    float* d = grad + r * C;
    if (has_ignore && target[r] == ignore) {
      for (int64_t c = 0; c < C; ++c) d[c] = 0.0f;
      continue;
    }
    int64_t t = target[r];
    if (t < 0) t = 0;
    if (t >= C) t = C - 1;
    float maximum = -INFINITY;
    for (int64_t c = 0; c < C; ++c) maximum = java_max(maximum, l[c]);
    for (int64_t c = 0; c < C; ++c) e[c] = (float)exp((double)(l[c] - maximum));
    const float s = shko_exact_sum(e, C, 1);
    for (int64_t c = 0; c < C; ++c) {
      float prob = e[c] / s;
      float hot = c == t ? 1.0f : 0.0f;
      d[c] = (prob - hot) * scale;
    }
  }
  free(e);
}

/* ------------------------------------------------------------------------------------------
 * Optimizers (TrainingParameter.java). Each stage function writes candidates only and returns
 * 0, or 1 when an intermediate is not finite / a bias correction or denominator is not
 * positive (the reference throws ArithmeticException before committing anything).
 * ------------------------------------------------------------------------------------------ */
#define FIN(v) do { if (!isfinite(v)) return 1; } while (0)

/* stageUpdate32 :622-672 */
int shko_sgd_stage(const float* p, const float* g, const float* m, float* p_out, float* m_out,
                   int64_t n, float lr, float momentum, float dampening, float weight_decay,
                   int nesterov, int has_momentum_slot, int64_t completed_steps) {
  const int first = completed_steps == 0;
  for (int64_t i = 0; i < n; ++i) {
    float pv = p[i];
    FIN(pv);
    float decay = weight_decay * pv;
    FIN(decay);
    float adjusted = g[i] + decay;
    FIN(adjusted);
    float selected = adjusted;
    if (momentum != 0.0f) {
      float um;
      if (first) um = adjusted;
      else {
        float mt = momentum * m[i];
        FIN(mt);
        float dg = (1.0f - dampening) * adjusted;
        FIN(dg);
        um = mt + dg;
      }
      FIN(um);
      m_out[i] = um;
      if (nesterov) {
        float look = momentum * um;
        FIN(look);
        selected = adjusted + look;
        FIN(selected);
      } else {
        selected = um;
      }
    } else if (has_momentum_slot) {
      m_out[i] = 0.0f;
    }
    float scaled = lr * selected;
    FIN(scaled);
    float cand = pv - scaled;
    FIN(cand);
    p_out[i] = cand;
  }
  return 0;
}

static int adam_tail(float base, float first, float second, float c1, float c2, float lr,
                     float eps, float* out);

/* stageAdaptive32 / stageAdaptiveElement32 :433-525; decoupled = AdamW. */
int shko_adam_stage(const float* p, const float* g, const float* m, const float* v, float* p_out,
                    float* m_out, float* v_out, int64_t n, float lr, float b1, float b2, float eps,
                    float decay, int decoupled, int64_t completed_steps) {
  const int64_t step = completed_steps + 1;
  float c1 = 1.0f - (float)pow((double)b1, (double)step);
  float c2 = 1.0f - (float)pow((double)b2, (double)step);
  if (!isfinite(c1) || c1 <= 0.0f || !isfinite(c2) || c2 <= 0.0f) return 1;
  float decay_factor = 1.0f;
  if (decoupled) {
    float scale = lr * decay;
    FIN(scale);
    decay_factor -= scale;
    FIN(decay_factor);
  }
  for (int64_t i = 0; i < n; ++i) {
    float pv = p[i];
    FIN(pv);
    float gradient, base;
    if (decoupled) {
      base = pv * decay_factor;
      FIN(base);
      gradient = g[i];
    } else {
      float dt = decay * pv;
      FIN(dt);
      gradient = g[i] + dt;
      FIN(gradient);
      base = pv;
    }
    float ft = b1 * m[i];
    FIN(ft);
    float fg = (1.0f - b1) * gradient;
    FIN(fg);
    float first = ft + fg;
    FIN(first);
    float sq = gradient * gradient;
    FIN(sq);
    float st = b2 * v[i];
    FIN(st);
    float sg = (1.0f - b2) * sq;
    FIN(sg);
    float second = st + sg;
    FIN(second);
    float cand;
    if (adam_tail(base, first, second, c1, c2, lr, eps, &cand)) return 1;
    m_out[i] = first;
    v_out[i] = second;
    p_out[i] = cand;
  }
  return 0;
}

/* The parameter candidate of one Adam element from its new moments (the tail of
 * stageAdaptiveElement32): p_out = base - (lr * (first / c1)) / ((float)sqrt(second / c2) + eps),
 * with the same finiteness checks. Shared by shko_adam_stage and shko_adam_apply. */
static int adam_tail(float base, float first, float second, float c1, float c2, float lr,
                     float eps, float* out) {
  float cf = first / c1;
  float cs = second / c2;
  FIN(cf);
  FIN(cs);
  float root = (float)sqrt((double)cs);
  FIN(root);
  float denom = root + eps;
  if (!isfinite(denom) || denom <= 0.0f) return 1;
  float numer = lr * cf;
  FIN(numer);
  float update = numer / denom;
  FIN(update);
  float cand = base - update;
  FIN(cand);
  *out = cand;
  return 0;
}

/* Adam's parameter candidates from given new moments m_new, v_new (for checking a device's
 * update arithmetic independently of its gradient): the base is p (coupled decay) or
 * p * (1 - lr * decay) (decoupled), then adam_tail. Returns 1 on a non-finite intermediate. */
int shko_adam_apply(const float* p, const float* m_new, const float* v_new, float* p_out,
                    int64_t n, float lr, float b1, float b2, float eps, float decay,
                    int decoupled, int64_t completed_steps) {
  const int64_t step = completed_steps + 1;
  float c1 = 1.0f - (float)pow((double)b1, (double)step);
  float c2 = 1.0f - (float)pow((double)b2, (double)step);
  if (!isfinite(c1) || c1 <= 0.0f || !isfinite(c2) || c2 <= 0.0f) return 1;
  float decay_factor = 1.0f;
  if (decoupled) {
    float scale = lr * decay;
    FIN(scale);
    decay_factor -= scale;
    FIN(decay_factor);
  }
  for (int64_t i = 0; i < n; ++i) {
    float base = p[i];
    FIN(base);
    if (decoupled) {
      base = base * decay_factor;
      FIN(base);
    }
    if (adam_tail(base, m_new[i], v_new[i], c1, c2, lr, eps, &p_out[i])) return 1;
  }
  return 0;
}

/* Canonical host publication (MetalBackendRuntime.copyToCanonicalHostBytes,
 * MetalBackendRuntime.java:360-398, with storageElementIndex :489-499): for every row-major
 * ordinal, the storage element is offset + sum(coordinate_a * stride_a) with the coordinates
 * peeled from the last axis; its `width` bytes are written in reverse (little-endian host ->
 * big-endian) order; BOOL elements must be 0 or 1. strides == NULL means dense row-major.
 * Returns 0, 1 for a non-canonical BOOL byte, 2 for a span outside src (nothing is promised
 * about dst after a non-zero return). */
int shko_canonical_bytes(const uint8_t* src, uint64_t src_bytes, int width, int boolean,
                         int rank, const int64_t* dims, const int64_t* strides, int64_t offset,
                         uint8_t* dst) {
  int64_t elements = 1;
  for (int a = 0; a < rank; ++a) elements *= dims[a];
  for (int64_t ordinal = 0; ordinal < elements; ++ordinal) {
    int64_t remaining = ordinal, storage = offset, dense_stride = 1;
    for (int a = rank - 1; a >= 0; --a) {
      const int64_t coordinate = remaining % dims[a];
      remaining /= dims[a];
      const int64_t stride = strides != NULL ? strides[a] : dense_stride;
      storage += coordinate * stride;
      dense_stride *= dims[a];
    }
    const uint64_t at = (uint64_t)storage * (uint64_t)width;
    if (at + (uint64_t)width > src_bytes) return 2;
    if (boolean) {
      if (src[at] != 0 && src[at] != 1) return 1;
      dst[ordinal] = src[at];
      continue;
    }
    for (int k = 0; k < width; ++k) dst[ordinal * width + k] = src[at + (uint64_t)(width - 1 - k)];
  }
  return 0;
}
