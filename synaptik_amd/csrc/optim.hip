// Fused, transactional SGD / Adam / AdamW parameter update over many tensors in one launch.
//
// Arithmetic restates TrainingParameter.stageUpdate32 (SGD, momentum, dampening, Nesterov,
// coupled weight decay; modules/training/.../TrainingParameter.java:622-672) and
// stageAdaptive32 / stageAdaptiveElement32 (Adam with coupled decay, AdamW with decoupled
// decay; TrainingParameter.java:433-525) operation by operation in binary32, with the same
// finiteness checks on every intermediate and candidate.
//
// The reference stages candidates on the host and commits them only if every element of every
// parameter passed its checks. On the device this is two streaming phases:
//   phase 0 (check): recompute every intermediate, OR DEV_NON_FINITE / DEV_NOT_POSITIVE into the
//                    program status word; nothing is written to parameters or slots;
//   phase 1 (apply): if the status word is clear, recompute and store parameter and slots.
// A failed step therefore leaves parameters and optimizer slots bit-for-bit unchanged, and the
// completed-step counter is advanced only by launch_step_commit when the status stays clear.
// Traffic: check reads p,g,m(,v); apply reads p,g,m(,v) and writes p,m(,v).
//
// With double-buffered parameters and slots one pass suffices:
//   phase 2 (stage): read the current p,g,m(,v), write every candidate to the other buffer set
//                    (pn,mn,vn) and flag failures; the host adopts the candidate set only when the
//                    run returns OK, so a failed step still commits nothing. Traffic 20 B (SGD
//                    momentum) / 28 B (Adam) per parameter instead of 32 / 44.
#include "common.h"
#include "kernels.h"
#include "optim_math.h"

namespace shk {
namespace {

constexpr int OPT_NT = 256;
constexpr int OPT_PER_THREAD = 4;
constexpr int64_t OPT_CHUNK = OPT_NT * OPT_PER_THREAD;

// Gradient accumulation (TrainingParameter.stageAccumulation:374-389, GradientMode):
//   kind 3  p = m + g with every candidate checked finite (m: accumulator, p: the step's
//           gradient buffer, rewritten in place);
//   kind 4  m = g, only if the status word is clear (commit of an ACCUMULATE run);
//   kind 5  m = 0, only if the status word is clear (accumulator emptied by a successful step).
__device__ void accumulation_block(const OptParams& p, const OptTensor& T, int64_t base) {
  if (p.kind != 3 && *(volatile const uint32_t*)p.status != 0u) return;
  bool ok = true;
#pragma unroll
  for (int q = 0; q < OPT_PER_THREAD; ++q) {
    const int64_t i = base + q * OPT_NT + threadIdx.x;
    if (i >= T.n) break;
    if (p.kind == 3) {
      const float c = T.m[i] + T.g[i];
      ok &= is_finite(c);
      T.p[i] = c;
    } else if (p.kind == 4) {
      T.m[i] = T.g[i];
    } else {
      T.m[i] = 0.0f;
    }
  }
  if (p.kind == 3) {
    const int bad = wave_or(ok ? 0 : 1);
    if (bad && (threadIdx.x & 63) == 0) atomicOr(p.status, (uint32_t)DEV_NON_FINITE);
  }
}

// Block `block` of the optimizer pass (OPT_NT threads; no block barrier, so a workgroup may run
// several blocks one after the other with identical results).
__device__ __forceinline__ void optimizer_block(const OptParams& p, int64_t block) {
  // Tensor of this block: the table holds each tensor's first block index in `start`.
  int t = 0;
  for (int i = 1; i < p.count; ++i)
    if (block >= p.t[i].start) t = i;
  const OptTensor T = p.t[t];
  if (p.kind >= 3) {
    accumulation_block(p, T, (block - T.start) * OPT_CHUNK);
    return;
  }
  if (p.phase == 1 && *(volatile const uint32_t*)p.status != 0u) return;
  const int64_t completed = *p.completed_steps;
  const bool first = completed == 0;
  Coeffs k{1.0f, 1.0f, 1.0f, true};
  if (p.kind != 0) k = adam_coeffs(p, completed + 1);
  const int64_t base = (block - T.start) * OPT_CHUNK;
  bool ok = k.ok;
  // Each thread owns 4 consecutive elements: 128-bit streaming loads and stores when all 4 exist
  // and every pointer is 16-byte aligned (device allocations and arena slots are), scalar
  // otherwise.
  const int64_t i0 = base + (int64_t)threadIdx.x * OPT_PER_THREAD;
  const bool vec = i0 + 3 < T.n &&
      ((reinterpret_cast<uintptr_t>(T.p) | reinterpret_cast<uintptr_t>(T.g) |
        reinterpret_cast<uintptr_t>(T.m) | reinterpret_cast<uintptr_t>(T.v) |
        reinterpret_cast<uintptr_t>(T.pn) | reinterpret_cast<uintptr_t>(T.mn) |
        reinterpret_cast<uintptr_t>(T.vn)) & 15u) == 0;
  float pv[4], gv[4], mv[4], vv[4], pc[4], mc[4], vc[4];
  const int cnt = vec ? 4 : (int)max<int64_t>(0, min<int64_t>(4, T.n - i0));
  if (vec) {
    *reinterpret_cast<float4*>(pv) = ld_stream(reinterpret_cast<const float4*>(T.p + i0));
    *reinterpret_cast<float4*>(gv) = ld_stream(reinterpret_cast<const float4*>(T.g + i0));
    if (T.m != nullptr) *reinterpret_cast<float4*>(mv) = ld_stream(reinterpret_cast<const float4*>(T.m + i0));
    if (p.kind != 0) *reinterpret_cast<float4*>(vv) = ld_stream(reinterpret_cast<const float4*>(T.v + i0));
  } else {
    for (int q = 0; q < cnt; ++q) {
      pv[q] = T.p[i0 + q];
      gv[q] = T.g[i0 + q];
      if (T.m != nullptr) mv[q] = T.m[i0 + q];
      if (p.kind != 0) vv[q] = T.v[i0 + q];
    }
  }
  float chk = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (q >= cnt) break;
    const float m0 = T.m != nullptr ? mv[q] : 0.0f;
    vc[q] = 0.0f;
    if (p.kind == 0) sgd_element(p, first, pv[q], gv[q], m0, pc[q], mc[q], chk);
    else adam_element(p, k, pv[q], gv[q], m0, vv[q], pc[q], mc[q], vc[q], chk);
  }
  ok = ok && chk == 0.0f;
  if (p.phase != 0) {
    float* dp = p.phase == 1 ? T.p : T.pn;
    float* dm = p.phase == 1 ? T.m : T.mn;
    float* dv = p.phase == 1 ? T.v : T.vn;
    if (vec) {
      st_stream(reinterpret_cast<float4*>(dp + i0), *reinterpret_cast<const float4*>(pc));
      if (dm != nullptr) st_stream(reinterpret_cast<float4*>(dm + i0), *reinterpret_cast<const float4*>(mc));
      if (p.kind != 0) st_stream(reinterpret_cast<float4*>(dv + i0), *reinterpret_cast<const float4*>(vc));
    } else {
      for (int q = 0; q < cnt; ++q) {
        dp[i0 + q] = pc[q];
        if (dm != nullptr) dm[i0 + q] = mc[q];
        if (p.kind != 0) dv[i0 + q] = vc[q];
      }
    }
  }
  if (p.phase != 1) {
    const int bad = wave_or(ok ? 0 : 1);
    if (bad && (threadIdx.x & 63) == 0)
      atomicOr(p.status, k.ok ? (uint32_t)DEV_NON_FINITE : (uint32_t)DEV_NOT_POSITIVE);
  }
}

__global__ void __launch_bounds__(OPT_NT) optimizer_kernel(OptParams p) {
  optimizer_block(p, (int64_t)blockIdx.x);
}

// The run's last launch (RunFinale): folded steps in program order, then the publication. The
// optimizer blocks run one after the other in this workgroup with their kernel's arithmetic;
// their failure flags are OR-ed into the status word by device-scope atomics, which the fence
// and barrier order before lane 0 reads the word back at device scope.
// Instantiated with and without the optimizer pass: a run without one launches a kernel with no
// optimizer code (and no private memory).
template <bool OPT>
__global__ void __launch_bounds__(OPT_NT) run_finale_kernel(RunFinale f) {
  __shared__ double dl[OPT_NT / 64];
  if (f.R > 0 && f.mean_first) ce_mean_block(f.row_loss, f.R, f.loss, dl);
  if (OPT && f.opt.count > 0) {
    int64_t blocks = 0;
    for (int i = 0; i < f.opt.count; ++i) blocks += (f.opt.t[i].n + OPT_CHUNK - 1) / OPT_CHUNK;
    for (int64_t b = 0; b < blocks; ++b) optimizer_block(f.opt, b);
  }
  if (f.R > 0 && !f.mean_first) ce_mean_block(f.row_loss, f.R, f.loss, dl);
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t v = atomicOr(f.status, 0u);  // the word as the device's atomics left it
    if (f.counter != nullptr && v == 0u) f.counter[0] = f.counter[0] + 1;
    f.host_word[0] = v;
    f.status[0] = 0u;
  }
}

__global__ void step_commit_kernel(int64_t* counter, const uint32_t* status) {
  if (threadIdx.x == 0 && blockIdx.x == 0 && *status == 0u) *counter = *counter + 1;
}

}  // namespace

namespace {
// Fills each tensor's first block index; returns the block count.
int64_t assign_blocks(OptParams& p) {
  int64_t blocks = 0;
  for (int i = 0; i < p.count; ++i) {
    p.t[i].start = blocks;
    blocks += (p.t[i].n + OPT_CHUNK - 1) / OPT_CHUNK;
  }
  return blocks;
}
}  // namespace

int64_t optimizer_blocks(const OptParams& in) {
  OptParams p = in;
  return assign_blocks(p);
}

hipError_t launch_optimizer(const OptParams& in, hipStream_t s) {
  OptParams p = in;
  const int64_t blocks = assign_blocks(p);
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(optimizer_kernel, dim3((unsigned)blocks), dim3(OPT_NT), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_run_finale(const RunFinale& in, hipStream_t s) {
  RunFinale f = in;
  if (f.opt.count > 0 && assign_blocks(f.opt) > RUN_FINALE_MAX_OPT_BLOCKS)
    return hipErrorInvalidValue;
  if (f.opt.count > 0)
    hipLaunchKernelGGL(run_finale_kernel<true>, dim3(1), dim3(OPT_NT), 0, s, f);
  else
    hipLaunchKernelGGL(run_finale_kernel<false>, dim3(1), dim3(OPT_NT), 0, s, f);
  return hipGetLastError();
}

hipError_t launch_step_commit(int64_t* counter, const uint32_t* status, hipStream_t s) {
  hipLaunchKernelGGL(step_commit_kernel, dim3(1), dim3(64), 0, s, counter, status);
  return hipGetLastError();
}

}  // namespace shk
