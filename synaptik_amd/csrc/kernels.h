// Host-side launch interface of the gfx950 kernels. Every launcher validates nothing itself:
// the program runtime (runtime.cpp) checks shapes, slot sizes and alignment before it calls
// them, so a launcher is only ever handed operands that match the grid it builds.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace shk {

// Status word bits written by kernels into the program's device status block.
enum DeviceStatus : uint32_t {
  DEV_OK = 0,
  DEV_NON_FINITE = 1,       // an optimizer intermediate or candidate was not finite
  DEV_INDEX_OUT_OF_BOUNDS = 2,  // a categorical target index lies outside the class extent
  DEV_NOT_POSITIVE = 4,     // an adaptive bias correction or denominator was not positive
  DEV_INVALID_BOOL = 8,     // a published BOOL element held a byte other than 0 or 1
};

// C[M,N] = op(A)[M,K] . op(B)[K,N] with a fused epilogue.
//   transA = 0: A is row-major [M,K] (K contiguous), transA = 1: A is stored [K,M].
//   transB = 0: B is row-major [K,N] (N contiguous), transB = 1: B is stored [N,K].
//   mode 0 (forward):  C = act(acc + bias)             (bias optional, act in Act)
//   mode 1 (backward): C = act_grad(act, acc, aux)       (aux = activation output y)
//   mode 2 (forward with its cotangent): C = act(acc + bias) as mode 0, and with aux = dY (the
//          upstream cotangent of C, leading dimension ldaux) also dz = act_grad(act, dY, C)
//          (same leading dimension); the optional column sum then sums dz, not C.
//   accumulate != 0:   the epilogue value is added to the existing C (gradient accumulation).
// Optimizer update fused into a GEMM epilogue that produces a weight gradient: the epilogue
// stages the candidate parameter and slots exactly as the streaming optimizer's phase 2 (same
// per-element arithmetic) from the freshly computed gradient, which is never stored. Enabled when
// pn != nullptr; p, m, v, pn, mn, vn are row-major [M, N] like C. Field names match OptParams so
// the shared element functions take either.
struct GemmUpdate {
  const float* p;
  const float* m;
  const float* v;
  float* pn;
  float* mn;
  float* vn;
  int kind;  // 0 SGD, 1 Adam, 2 AdamW
  int nesterov, has_momentum_slot;
  float lr, momentum, dampening, weight_decay;
  float beta1, beta2, eps;
  const int64_t* completed_steps;
  uint32_t* status;
};

struct GemmParams {
  const float* A;
  const float* B;
  float* C;
  const float* bias;
  const float* aux;
  int64_t M, N, K;
  int64_t lda, ldb, ldc, ldaux;
  int transA, transB;
  int act, mode, accumulate;
  // Split-K (set by launch_gemm, not by callers): block row y handles K slice
  // [y*kchunk, min(K, (y+1)*kchunk)) and writes raw partial sums to partial[y][M][N].
  float* partial;
  int64_t kchunk;
  // Optional fused column sum of the stored C (SUM_TO_SHAPE for a bias gradient): colsum[N]
  // receives the sum over all M rows; colsum_partial is launch_gemm's workspace.
  float* colsum;
  double* colsum_partial;
  // mode 2: the cotangent of the activation input, [M, N] with leading dimension ldaux
  float* dz;
  // Optional fused optimizer update (C is then not written and may be null; requires ldc == N,
  // mode 0, no bias, no activation, no accumulate, no column sum).
  GemmUpdate upd;
};
// `workspace` holds at least gemm_workspace_floats(M, N, K) floats (split-K partials); it may be
// null when that is 0.
hipError_t launch_gemm(const GemmParams& p, float* workspace, hipStream_t s);
int64_t gemm_workspace_floats(int64_t M, int64_t N, int64_t K, bool colsum = false);
// Finishes a column sum from P partial rows (binary64, fixed order) into out[N].
hipError_t launch_colsum_finish(const double* partial, float* out, int64_t P, int64_t N,
                                hipStream_t s);

// Column sums of X[R,N] (row stride ldx) into out[N]; out = (float)(sum * scale_num / scale_den)
// with the sum accumulated in binary64. Used for SUM_TO_SHAPE (bias gradients) and MEAN.
// When accumulate != 0 the result is added to out.
hipError_t launch_colsum(const float* x, float* out, int64_t R, int64_t N, int64_t ldx,
                         double divisor, int accumulate, double* partial, hipStream_t s);
int64_t colsum_partial_doubles(int64_t R, int64_t N);

// Row reductions over the last axis of X[R,C]: kind 0 SUM, 1 MEAN, 2 MAX, 3 LOG_SUM_EXP.
hipError_t launch_row_reduce(const float* x, float* out, int64_t R, int64_t C, int kind,
                             hipStream_t s);

// Whole-tensor reductions: kind 0 SUM, 1 MEAN, 2 MAX. Two deterministic passes through
// `partial` (at least reduce_all_partial_doubles(n) doubles).
hipError_t launch_reduce_all(const float* x, float* out, int64_t n, int kind, double* partial,
                             hipStream_t s);
int64_t reduce_all_partial_doubles(int64_t n);

// Row softmax / log-softmax over the last axis with the reference's special-value classes;
// optionally also writes the per-row log-sum-exp.
hipError_t launch_softmax_fwd(const float* x, float* y, float* lse, int64_t R, int64_t C,
                              int log_softmax, hipStream_t s);
// dX = y (.) (g - sum(g (.) y)) + rowscale[r] * y   (rowscale optional: LOG_SUM_EXP cotangent
// folded in, e.g. dm/R for a MEAN over the row LSE values; rowscale_const used if ptr null).
hipError_t launch_softmax_bwd(const float* y, const float* g, float* dx, int64_t R, int64_t C,
                              const float* rowscale, float rowscale_const, hipStream_t s);
// dX = g[r] * exp(x - lse[r])  (LOG_SUM_EXP gradient) with g a per-row cotangent or constant.
hipError_t launch_lse_bwd(const float* x, const float* lse, const float* g, float gconst,
                          float* dx, int64_t R, int64_t C, hipStream_t s);

// Squared error over n elements, MEAN (loss = sum((p-t)^2) / n, grad = ((p-t)*2) * (g/n)) or
// SUM (loss = sum((p-t)^2), grad = ((p-t)*2) * g).
hipError_t launch_mse(const float* p, const float* t, float* loss, float* grad, int64_t n,
                      float g, int reduction_sum, double* partial, hipStream_t s);
int64_t mse_partial_doubles(int64_t n);

// Index categorical cross-entropy with logits [R,C], integer targets [R] (int32 or int64),
// MEAN over non-ignored samples; grad = (softmax - onehot(clamp(t))) * (g / count).
hipError_t launch_index_ce(const float* logits, const void* target, int target_is_64,
                           float* loss, float* grad, int64_t R, int64_t C, int has_ignore,
                           int64_t ignore_index, float g, double* partial, uint32_t* status,
                           hipStream_t s);
int64_t index_ce_partial_doubles(int64_t R);

// Fused classifier head (J <= 16 classes, MEAN index cross-entropy without an ignore index):
// logits = H . W^T + b, row_loss[r], dz = (softmax - onehot) * (g / R) and, when dx is set,
// dx = act_grad(act, dz . W, H), each bit-identical to the unfused row-dot GEMM, CE and small-K
// GEMM sequence. H [R, K], W [J, K], bias [J] (optional), logits [R, J] (optional), dz [R, J].
struct CeHeadParams {
  const float* H;
  const float* W;
  const float* bias;
  const void* target;
  float* logits;
  float* dz;
  float* dx;
  float* row_loss;
  uint32_t* status;
  int64_t R, K;
  int J, act, target_is_64, vec;
  float g;
};
hipError_t launch_ce_head(const CeHeadParams& p, hipStream_t s);
// loss[0] = MEAN of row_loss[0 .. R) (binary64 sum, one rounding, divided by R).
hipError_t launch_ce_head_finish(const float* row_loss, int64_t R, float* loss, hipStream_t s);

// Interpreted fused elementwise chain (see pointwise.hip for the instruction set).
struct PwInstr {
  uint8_t op, dst, a, b;
  uint8_t c, pad0, pad1, pad2;
  float imm;
};
constexpr int PW_MAX_INPUTS = 6;
constexpr int PW_MAX_OUTPUTS = 2;
constexpr int PW_MAX_INSTR = 48;
struct PwParams {
  const float* in[PW_MAX_INPUTS];
  int64_t in_mode[PW_MAX_INPUTS];  // 0 full [R,C], 1 row vector [C], 2 column [R], 3 scalar
  float* out[PW_MAX_OUTPUTS];
  int64_t R, C;
  int n_instr;
  PwInstr code[PW_MAX_INSTR];
};
hipError_t launch_pointwise(const PwParams& p, hipStream_t s);

// Multi-tensor optimizer. Each entry is one parameter tensor with its gradient and slots.
constexpr int OPT_MAX_TENSORS = 16;
struct OptTensor {
  float* p;
  const float* g;
  float* m;
  float* v;
  float* pn;  // phase 2: candidate parameter / slot buffers (the other half of a double buffer)
  float* mn;
  float* vn;
  int64_t n;
  int64_t start;  // first block of this tensor in the launch
};
struct OptParams {
  OptTensor t[OPT_MAX_TENSORS];
  int count;
  int64_t total;
  int kind;        // 0 SGD, 1 Adam (coupled decay), 2 AdamW (decoupled decay),
                   // 3 accumulate-sum, 4 commit accumulator, 5 clear accumulator (gated)
  int phase;       // 0 check (validate every intermediate), 1 apply (commit if status clear),
                   // 2 stage (one pass: write candidates to pn/mn/vn, flag failures)
  float lr, momentum, dampening, weight_decay;  // SGD
  int nesterov, has_momentum_slot;
  float beta1, beta2, eps;                       // Adam
  const int64_t* completed_steps;  // device counter of prior successful updates
  uint32_t* status;
};
hipError_t launch_optimizer(const OptParams& p, hipStream_t s);
// Blocks of 1024 elements that launch_optimizer would run for `p` (no launch).
int64_t optimizer_blocks(const OptParams& p);
// The last launch of a run, one workgroup: the program's folded trailing steps in program order
// -- the loss MEAN of a fused classifier head (ce_mean: row_loss[0 .. R) into loss[0], when
// R > 0) and a staged optimizer pass of at most RUN_FINALE_MAX_OPT_BLOCKS blocks (opt_count > 0),
// each with the arithmetic of its own kernel -- then the status publication: the step commit
// when a counter is given (it advances when the word is clear), the copy into the pinned host
// word and the clear for the next run.
constexpr int64_t RUN_FINALE_MAX_OPT_BLOCKS = 8;
struct RunFinale {
  const float* row_loss;
  int64_t R;
  float* loss;
  int mean_first;  // the MEAN precedes the optimizer pass in program order
  OptParams opt;   // opt.count == 0: no optimizer pass
  uint32_t* status;
  uint32_t* host_word;
  int64_t* counter;
};
hipError_t launch_run_finale(const RunFinale& f, hipStream_t s);
// Increments the completed-step counter when the status word is clear.
hipError_t launch_step_commit(int64_t* counter, const uint32_t* status, hipStream_t s);

hipError_t launch_fill(float* x, int64_t n, float value, hipStream_t s);
hipError_t launch_fill_u32(uint32_t* x, int64_t n, uint32_t value, hipStream_t s);
hipError_t launch_copy(const float* src, float* dst, int64_t n, hipStream_t s);
// Canonical publication geometry of a strided view (element units, row-major ordinals).
constexpr int CANONICAL_MAX_RANK = 16;
struct CanonicalGeometry {
  int64_t dims[CANONICAL_MAX_RANK];
  int64_t strides[CANONICAL_MAX_RANK];
  int64_t offset;
  int32_t rank;
};
// Packs `elements` elements of `width` bytes (1, 2, 4, 8) from src into dense big-endian bytes at
// dst; g == nullptr means src is dense from element 0 (src and dst 16-byte aligned). boolean: the
// elements are BOOL bytes, any value other than 0 / 1 ORs DEV_INVALID_BOOL into *status.
hipError_t launch_canonical_pack(const void* src, void* dst, int64_t elements, int width,
                                 int boolean, const CanonicalGeometry* g, uint32_t* status,
                                 hipStream_t s);

// ORs DEV_INVALID_BOOL into *status when any of the `elements` logical BOOL bytes of the view
// g over src is neither 0 nor 1; reads only.
hipError_t launch_bool_validate(const void* src, int64_t elements, const CanonicalGeometry& g,
                                uint32_t* status, hipStream_t s);

// Y[C,R] = X[R,C]^T
hipError_t launch_transpose(const float* x, float* y, int64_t R, int64_t C, hipStream_t s);

}  // namespace shk
