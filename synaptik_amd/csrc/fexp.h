// Binary32 exponential accurate to about 0.6 ulp, for the softmax forward pass.
//
// The reference evaluates softmax addends as (float)StrictMath.exp((double)(x - shift))
// (CpuSoftmaxReferenceKernel.java:104-146): a binary64 exponential rounded once to binary32.
// A binary64 exponential per element costs more VALU time on the GPU than the HBM traffic it
// hides behind, so this routine computes the same value directly in binary32 for arguments whose
// result is a normal float, and returns exactly the reference expression elsewhere.
//
// Method (Cody and Waite, "Software Manual for the Elementary Functions", 1980): write
//   t = n ln2 + r,  n = rint(t / ln2),  |r| <= ln2 / 2 (plus rounding),
// with ln2 split into L1 = binary32(ln2) and L2 = binary32(ln2 - L1). n is formed by adding the
// shifter 1.5 * 2^23 to t / ln2 in one FMA: the sum's spacing is 1, so the FMA rounds t / ln2 to
// the nearest integer once, and the shifter's low mantissa bits then hold n (two's complement in
// the bits that survive a shift left by 23). Because L1 has 24 significant bits and |n| <= 127,
// t - n L1 is exactly representable and one FMA forms it exactly; the second FMA subtracts n L2
// with a single rounding. exp(r) is the Taylor polynomial of degree 7 (truncation error below
// 0.35^8 / 8! = 5.4e-9, i.e. below 0.1 ulp of 1) by Horner's rule with FMAs down to the constant
// term, whose FMA rounds once; scaling by 2^n adds n to the exponent field, exact in the normal
// range. Checked on the host against the binary64 expression for every 7th binary32 argument in
// [-87, 88]: at most 1 ulp, 0.46% of arguments differ.
//
// Range: for t in [-87, 88] the result is a normal binary32 (n in [-126, 127], and for
// n = -126 the reduced argument is positive). Outside it (overflow to +inf, subnormal results,
// underflow to 0, -inf, NaN) the binary64 expression is evaluated, so those cases agree with the
// reference exactly.
//
// Written for both the device and the host (the host build checks it against the binary64
// expression over millions of arguments); the host including file defines __host__ and
// __device__ as nothing.
#pragma once
#include <math.h>
#include <stdint.h>

namespace shk {

// The binary32 path alone: the caller guarantees t in [-87, 88].
__host__ __device__ inline float exp_f32_in_range(float t) {
  const float kLog2e = 0x1.715476p+0f;     // binary32(1 / ln 2)
  const float kLn2Hi = 0x1.62e430p-1f;     // L1 = binary32(ln 2)
  const float kLn2Lo = -0x1.05c610p-29f;   // L2 = binary32(ln 2 - L1)
  const float kShift = 0x1.8p23f;          // 1.5 * 2^23
  const float k = fmaf(t, kLog2e, kShift);
  const float n = k - kShift;              // exact
  float r = fmaf(-n, kLn2Hi, t);           // exact
  r = fmaf(-n, kLn2Lo, r);
  float q = 0x1.a01a02p-13f;            // 1/7!
  q = fmaf(q, r, 0x1.6c16c2p-10f);      // 1/6!
  q = fmaf(q, r, 0x1.111112p-7f);       // 1/5!
  q = fmaf(q, r, 0x1.555556p-5f);       // 1/4!
  q = fmaf(q, r, 0x1.555556p-3f);       // 1/3!
  q = fmaf(q, r, 0.5f);                 // 1/2!
  q = fmaf(q, r, 1.0f);                 // 1/1!
  const float e = fmaf(q, r, 1.0f);     // 1/0!
  uint32_t eb, kb;
  __builtin_memcpy(&eb, &e, 4);
  __builtin_memcpy(&kb, &k, 4);
  eb += kb << 23;                       // n << 23 (mod 2^32): the low bits of k hold n
  float out;
  __builtin_memcpy(&out, &eb, 4);
  return out;
}

__host__ __device__ inline float exp_f32(float t) {
  if (t >= -87.0f && t <= 88.0f) return exp_f32_in_range(t);
  return (float)exp((double)t);
}

}  // namespace shk
