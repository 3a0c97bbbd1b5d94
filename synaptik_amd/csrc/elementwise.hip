// Fused elementwise chains and SUM/MEAN/MAX reductions for gfx950.
//
// Pointwise: the reference fuses elementwise/activation chains into one generated kernel per
// chain (CPU: CpuPointwiseGeneratedKernelTest; Metal: SynaptikPointwiseFusionKernelSource.h,
// a runtime-generated instruction-list unit). Here one precompiled kernel interprets a short
// register-machine program held in the kernel arguments: the opcode stream is wave-uniform, so
// every branch is scalar and the kernel stays HBM-bound with one read per input and one write
// per output, four elements per thread through 128-bit accesses.
//
// Reductions: SUM/MEAN/SUM_TO_SHAPE are exact in the reference (fixed-width limb accumulation
// rounded once, CpuExactSumEmitter.java:4-12, CpuAggregateEmitter.java:18-20). The GPU
// accumulates binary32 inputs in binary64 through a fixed-shape tree (wave shuffles, then LDS,
// then a second deterministic pass) and rounds once; that equals the exactly rounded sum
// unless the binary64 accumulation error crosses a binary32 rounding boundary. MAX follows
// Java Math.max (NaN wins, +0.0 beats -0.0).
#include "common.h"
#include "kernels.h"
#include <algorithm>

namespace shk {
namespace {

enum PwOp : uint8_t {
  PW_LOAD = 0,     // r[dst] = in[a]
  PW_CONST = 1,    // r[dst] = imm
  PW_ADD = 2, PW_SUB = 3, PW_MUL = 4, PW_DIV = 5,
  PW_NEG = 6,
  PW_RELU = 7, PW_TANH = 8, PW_SIGMOID = 9,
  PW_EXP = 10, PW_LOG = 11,
  PW_RELU_GRAD = 12,     // r[dst] = r[a] > 0 ? r[b] : 0          (WHERE(x > 0, g, 0))
  PW_TANH_GRAD = 13,     // r[dst] = r[b] * (1 - r[a]*r[a])      (a = y, b = g)
  PW_SIGMOID_GRAD = 14,  // r[dst] = (r[b] * r[a]) * (1 - r[a])  (a = y, b = g)
  PW_GT = 15,            // r[dst] = r[a] > r[b] ? 1 : 0
  PW_WHERE = 16,         // r[dst] = r[c] != 0 ? r[a] : r[b]
  PW_STORE = 17,         // out[dst] = r[a]
  PW_MAX = 18,           // Java Math.max
  PW_SQRT = 19,
};
constexpr int PW_REGS = 8;

// Binary64-evaluated transcendentals kept out of line: they are rare in chains, and inlining
// them into every interpreter case inflates the register allocation of the whole kernel.
__device__ __noinline__ float pw_tanh(float a) { return tanh_f(a); }
__device__ __noinline__ float pw_sigmoid(float a) { return sigmoid_f(a); }
__device__ __noinline__ float pw_exp(float a) { return (float)exp((double)a); }
__device__ __noinline__ float pw_log(float a) { return (float)log((double)a); }
__device__ __noinline__ float pw_sqrt(float a) { return (float)sqrt((double)a); }

// One instruction's value from its operands (a, b, c registers; imm for CONST). Shared by the
// interpreter (op known at run time) and the single-op kernels (op a template constant).
__device__ __forceinline__ float pw_op(int op, float a, float b, float c, float imm) {
  switch (op) {
    case PW_CONST: return imm;
    case PW_ADD: return a + b;
    case PW_SUB: return a - b;
    case PW_MUL: return a * b;
    case PW_DIV: return a / b;
    case PW_NEG: return -a;
    case PW_RELU: return relu_f(a);
    case PW_TANH: return pw_tanh(a);
    case PW_SIGMOID: return pw_sigmoid(a);
    case PW_EXP: return pw_exp(a);
    case PW_LOG: return pw_log(a);
    case PW_RELU_GRAD: return act_grad(ACT_RELU, b, a);
    case PW_TANH_GRAD: return act_grad(ACT_TANH, b, a);
    case PW_SIGMOID_GRAD: return act_grad(ACT_SIGMOID, b, a);
    case PW_GT: return a > b ? 1.0f : 0.0f;
    case PW_WHERE: return (c != 0.0f) ? a : b;
    case PW_STORE: return a;
    case PW_MAX: return java_max(a, b);
    case PW_SQRT: return pw_sqrt(a);
    default: return 0.0f;
  }
}

// Single-op chains (LOAD x [, LOAD y], OP, STORE) over full-shape, 16-byte aligned operands (out
// may be one of them: each element is read before it is written): out
// = OP(x, y) element by element with the interpreter's arithmetic (pw_op), streaming 16-byte
// accesses, two groups of four per thread and iteration, no interpreter.
template <int OP, bool BIN>
__global__ void __launch_bounds__(256) pw_single_kernel(const float* x,
                                                        const float* y,
                                                        float* out, int64_t n) {
  const int64_t n4 = n / 4;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < n4; q += 2 * stride) {
    const bool two = q + stride < n4;
    const float4 xa = ld_stream(reinterpret_cast<const float4*>(x) + q);
    const float4 ya = BIN ? ld_stream(reinterpret_cast<const float4*>(y) + q) : xa;
    float4 xb = xa, yb = ya;
    if (two) {
      xb = ld_stream(reinterpret_cast<const float4*>(x) + q + stride);
      yb = BIN ? ld_stream(reinterpret_cast<const float4*>(y) + q + stride) : xb;
    }
    st_stream(reinterpret_cast<float4*>(out) + q,
              make_float4(pw_op(OP, xa.x, ya.x, 0.f, 0.f), pw_op(OP, xa.y, ya.y, 0.f, 0.f),
                          pw_op(OP, xa.z, ya.z, 0.f, 0.f), pw_op(OP, xa.w, ya.w, 0.f, 0.f)));
    if (two)
      st_stream(reinterpret_cast<float4*>(out) + q + stride,
                make_float4(pw_op(OP, xb.x, yb.x, 0.f, 0.f), pw_op(OP, xb.y, yb.y, 0.f, 0.f),
                            pw_op(OP, xb.z, yb.z, 0.f, 0.f), pw_op(OP, xb.w, yb.w, 0.f, 0.f)));
  }
  if (blockIdx.x == 0 && threadIdx.x < n - n4 * 4) {
    const int64_t i = n4 * 4 + threadIdx.x;
    out[i] = pw_op(OP, x[i], BIN ? y[i] : x[i], 0.f, 0.f);
  }
}

// Loads input k for the 4-element group starting at e0 (cnt valid elements) into v.
__device__ __forceinline__ void pw_load4(const PwParams& p, int k, int64_t e0, int cnt, float (&v)[4]) {
  const float* src = p.in[k];
  switch (p.in_mode[k]) {
    case 0:
      if (cnt == 4 && (reinterpret_cast<uintptr_t>(src + e0) & 15u) == 0) {
        const float4 t = ld_stream(reinterpret_cast<const float4*>(src + e0));
        v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
      } else {
        for (int q = 0; q < cnt; ++q) v[q] = src[e0 + q];
      }
      break;
    case 3: {
      const float t = src[0];
      v[0] = v[1] = v[2] = v[3] = t;
      break;
    }
    default: {
      // one division per group, then walk (row, col) forward
      int64_t row = e0 / p.C, col = e0 - row * p.C;
      for (int q = 0; q < cnt; ++q) {
        v[q] = p.in_mode[k] == 1 ? src[col] : src[row];
        if (++col == p.C) { col = 0; ++row; }
      }
    }
  }
}

// The interpreter's register file lives in LDS: register k of thread t holds its 4 elements at
// regs[k][t*4 .. t*4+3]. Any register index is then just an address (no dynamically indexed
// VGPR array, no scratch), and each operand access is one 128-bit LDS access per lane.
constexpr int PW_NT = 256;
struct PwRegs {
  float4 v[PW_REGS][PW_NT];
};

__device__ __forceinline__ void pw_exec(const PwParams& p, PwRegs& R, int64_t e0, int cnt,
                                        float (&outv)[PW_MAX_OUTPUTS][4]) {
  const int t = threadIdx.x;
  for (int pc = 0; pc < p.n_instr; ++pc) {
    const PwInstr ins = p.code[pc];
    float4& d4 = R.v[ins.dst & (PW_REGS - 1)][t];
    if (ins.op == PW_LOAD) {
      float v[4] = {0.f, 0.f, 0.f, 0.f};
      pw_load4(p, ins.a % PW_MAX_INPUTS, e0, cnt, v);
      d4 = make_float4(v[0], v[1], v[2], v[3]);
      continue;
    }
    const float4 a4 = R.v[ins.a & (PW_REGS - 1)][t];
    const float4 b4 = R.v[ins.b & (PW_REGS - 1)][t];
    const float a[4] = {a4.x, a4.y, a4.z, a4.w};
    const float b[4] = {b4.x, b4.y, b4.z, b4.w};
    float c[4] = {0.f, 0.f, 0.f, 0.f};
    if (ins.op == PW_WHERE) {
      const float4 c4 = R.v[ins.c & (PW_REGS - 1)][t];
      c[0] = c4.x; c[1] = c4.y; c[2] = c4.z; c[3] = c4.w;
    }
    float d[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) d[q] = pw_op(ins.op, a[q], b[q], c[q], ins.imm);
    if (ins.op == PW_STORE) {
      float* o = outv[ins.dst & 1];
      o[0] = d[0]; o[1] = d[1]; o[2] = d[2]; o[3] = d[3];
    } else {
      d4 = make_float4(d[0], d[1], d[2], d[3]);
    }
  }
}

__global__ void __launch_bounds__(PW_NT) pointwise_kernel(PwParams p) {
  __shared__ PwRegs regs;
  const int64_t n = p.R * p.C;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x * 4;
  for (int64_t e0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4; e0 < n; e0 += stride) {
    const int cnt = (int)min<int64_t>(4, n - e0);
    float outv[PW_MAX_OUTPUTS][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    pw_exec(p, regs, e0, cnt, outv);
    // Stores: vectorized when the group is complete and aligned.
#pragma unroll
    for (int o = 0; o < PW_MAX_OUTPUTS; ++o) {
      if (p.out[o] == nullptr) continue;
      float* dst = p.out[o] + e0;
      if (cnt == 4 && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
        st_stream(reinterpret_cast<float4*>(dst), make_float4(outv[o][0], outv[o][1], outv[o][2], outv[o][3]));
      } else {
        for (int q = 0; q < cnt; ++q) dst[q] = outv[o][q];
      }
    }
  }
}

__global__ void fill_kernel(float* x, int64_t n, float v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    x[i] = v;
}
__global__ void fill_u32_kernel(uint32_t* x, int64_t n, uint32_t v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    x[i] = v;
}
// One float4 per thread, streamed past the caches: many short workgroups keep the most bytes
// in flight per CU (measured on MI355X: 6.7 TB/s for a 1 GiB copy, against 5.2-5.8 TB/s for
// grid-stride loops and 5.2 TB/s for a device-to-device hipMemcpy).
__global__ void __launch_bounds__(256) copy_vec_kernel(const float4* __restrict__ s,
                                                       float4* __restrict__ d, int64_t n4) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n4) st_stream(&d[i], ld_stream(&s[i]));
}
__global__ void copy_kernel(const float* __restrict__ s, float* __restrict__ d, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    d[i] = s[i];
}

// Column sums, pass 1: block (cx, ry) sums a 64-column x `rows`-row panel; each of the 4 waves
// walks a quarter of the panel's rows with lanes on consecutive columns (coalesced 256 B rows).
// The panel height is chosen per call so that a launch has ~1024 blocks even for short inputs.
constexpr int CS_COLS = 64;
constexpr int64_t CS_TARGET_BLOCKS = 1024;
int64_t colsum_rows_per_panel(int64_t R, int64_t N) {
  const int64_t colblocks = (N + CS_COLS - 1) / CS_COLS;
  const int64_t panels = std::max<int64_t>(1, (CS_TARGET_BLOCKS + colblocks - 1) / colblocks);
  int64_t rows = (R + panels - 1) / panels;
  rows = std::max<int64_t>(64, ((rows + 3) / 4) * 4);
  return rows;
}
__global__ void __launch_bounds__(256) colsum_pass1(const float* __restrict__ x, double* part,
                                                   int64_t R, int64_t N, int64_t ldx, int64_t rows) {
  __shared__ double lds[4][CS_COLS];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t col = (int64_t)blockIdx.x * CS_COLS + lane;
  const int64_t r0 = (int64_t)blockIdx.y * rows;
  double s = 0.0;
  if (col < N) {
    const int64_t rend = min<int64_t>(R, r0 + rows);
    for (int64_t r = r0 + w; r < rend; r += 4) s += (double)x[r * ldx + col];
  }
  lds[w][lane] = s;
  __syncthreads();
  if (w == 0 && col < N)
    part[(int64_t)blockIdx.y * N + col] = ((lds[0][lane] + lds[1][lane]) + lds[2][lane]) + lds[3][lane];
}
// Pass 1 for 16-byte-aligned rows (N and ldx multiples of 4, x 16-byte aligned): each lane owns
// four adjacent columns and reads them with one streaming 16-byte load per row, so a wave moves
// 1 KiB per row and a block covers 256 columns. Panels, row assignment (rows r0 + w, r0 + w + 4,
// ...) and the combination order are those of colsum_pass1, so both write identical partials.
__global__ void __launch_bounds__(256) colsum_pass1_v4(const float* __restrict__ x, double* part,
                                                      int64_t R, int64_t N, int64_t ldx,
                                                      int64_t rows) {
  __shared__ double lds[4][4 * CS_COLS];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t col = ((int64_t)blockIdx.x * CS_COLS + lane) * 4;
  const int64_t r0 = (int64_t)blockIdx.y * rows;
  double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
  if (col < N) {
    const int64_t rend = min<int64_t>(R, r0 + rows);
#pragma unroll 4
    for (int64_t r = r0 + w; r < rend; r += 4) {
      const float4 v = ld_stream(reinterpret_cast<const float4*>(x + r * ldx + col));
      s0 += (double)v.x;
      s1 += (double)v.y;
      s2 += (double)v.z;
      s3 += (double)v.w;
    }
  }
  lds[w][4 * lane + 0] = s0;
  lds[w][4 * lane + 1] = s1;
  lds[w][4 * lane + 2] = s2;
  lds[w][4 * lane + 3] = s3;
  __syncthreads();
  const int c = threadIdx.x;  // one column of the block's 256 per thread
  const int64_t gc = (int64_t)blockIdx.x * 4 * CS_COLS + c;
  if (gc < N)
    part[(int64_t)blockIdx.y * N + gc] = ((lds[0][c] + lds[1][c]) + lds[2][c]) + lds[3][c];
}
// Column sums of a narrow input in one launch (N <= CS_SMALL_MAX_N, R <= CS_SMALL_MAX_R): block
// x sums 64 columns over all R rows with 16 waves (wave w: rows w, w + 16, ..., eight loads in
// flight), the waves' binary64 sums are added in wave order through LDS and finished as
// colsum_pass2 does.
constexpr int64_t CS_SMALL_MAX_N = 256;
constexpr int64_t CS_SMALL_MAX_R = 32768;
__global__ void __launch_bounds__(1024) colsum_small(const float* __restrict__ x, float* out,
                                                    int64_t R, int64_t N, int64_t ldx,
                                                    double divisor, int accumulate) {
  __shared__ double lds[16][CS_COLS];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t col = (int64_t)blockIdx.x * CS_COLS + lane;
  double s = 0.0;
  if (col < N) {
    int64_t r = w;
    for (; r + 7 * 16 < R; r += 8 * 16) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = x[(r + u * 16) * ldx + col];
#pragma unroll
      for (int u = 0; u < 8; ++u) s += (double)v[u];
    }
    for (; r < R; r += 16) s += (double)x[r * ldx + col];
  }
  lds[w][lane] = s;
  __syncthreads();
  if (w == 0 && col < N) {
    double t = lds[0][lane];
#pragma unroll
    for (int i = 1; i < 16; ++i) t += lds[i][lane];
    float v = (float)(t / divisor);
    if (accumulate) v = out[col] + v;
    out[col] = v;
  }
}
// Column sums, pass 2: block x finishes 64 columns; wave w adds partial rows w, w + 4, ... in
// two interleaved chains (independent loads in flight), then the chains and the four waves are
// combined in a fixed order, so results are run-to-run identical.
__global__ void __launch_bounds__(256) colsum_pass2(const double* part, float* out, int64_t P,
                                                    int64_t N, double divisor, int accumulate) {
  __shared__ double lds[4][CS_COLS];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t col = (int64_t)blockIdx.x * CS_COLS + lane;
  double s0 = 0.0, s1 = 0.0;
  if (col < N) {
    int64_t i = w;
    for (; i + 4 < P; i += 8) {
      s0 += part[i * N + col];
      s1 += part[(i + 4) * N + col];
    }
    if (i < P) s0 += part[i * N + col];
  }
  lds[w][lane] = s0 + s1;
  __syncthreads();
  if (w == 0 && col < N) {
    const double s = ((lds[0][lane] + lds[1][lane]) + lds[2][lane]) + lds[3][lane];
    float v = (float)(s / divisor);
    if (accumulate) v = out[col] + v;
    out[col] = v;
  }
}

// Row reductions: one workgroup per row, binary64 accumulation for SUM/MEAN/LSE.
template <int NT>
__global__ void __launch_bounds__(NT) row_reduce_kernel(const float* __restrict__ x, float* out,
                                                        int64_t C, int kind) {
  __shared__ double dl[NT / 64];
  __shared__ float fl[NT / 64];
  const float* row = x + (int64_t)blockIdx.x * C;
  if (kind == 2 || kind == 3) {
    float m = -INFINITY;
    for (int64_t c = threadIdx.x; c < C; c += NT) m = java_max(m, row[c]);
    m = block_max<NT>(m, fl);
    if (kind == 2) {
      if (threadIdx.x == 0) out[blockIdx.x] = C == 0 ? -INFINITY : m;
      return;
    }
    // LOG_SUM_EXP: shifted exponentials, one logarithm (CpuLogSumExpEmitter.java:4-9).
    const float shift = (m == INFINITY || m == -INFINITY) ? 0.0f : m;
    double s = 0.0;
    for (int64_t c = threadIdx.x; c < C; c += NT) s += (double)(float)exp((double)(row[c] - shift));
    s = block_sum<NT>(s, dl);
    if (threadIdx.x == 0) {
      float r;
      if (m != m) r = m;
      else if (m == INFINITY) r = INFINITY;
      else r = shift + (float)log((double)(float)s);
      out[blockIdx.x] = r;
    }
    return;
  }
  double s = 0.0;
  for (int64_t c = threadIdx.x; c < C; c += NT) s += (double)row[c];
  s = block_sum<NT>(s, dl);
  if (threadIdx.x == 0) out[blockIdx.x] = kind == 1 ? (float)(s / (double)C) : (float)s;
}

// Whole-tensor reductions in two deterministic passes.
constexpr int RA_BLOCKS = 1024;
__global__ void __launch_bounds__(256) reduce_all_pass1(const float* __restrict__ x, int64_t n,
                                                       int kind, double* part) {
  __shared__ double dl[4];
  __shared__ float fl[4];
  const int64_t stride = (int64_t)gridDim.x * 256;
  if (kind == 2) {
    float m = -INFINITY;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) m = java_max(m, x[i]);
    m = block_max<256>(m, fl);
    if (threadIdx.x == 0) part[blockIdx.x] = (double)m;
    return;
  }
  double s = 0.0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) s += (double)x[i];
  s = block_sum<256>(s, dl);
  if (threadIdx.x == 0) part[blockIdx.x] = s;
}
__global__ void __launch_bounds__(256) reduce_all_pass2(const double* part, int P, int64_t n,
                                                       int kind, float* out) {
  __shared__ double dl[4];
  __shared__ float fl[4];
  if (kind == 2) {
    float m = -INFINITY;
    for (int i = threadIdx.x; i < P; i += 256) m = java_max(m, (float)part[i]);
    m = block_max<256>(m, fl);
    if (threadIdx.x == 0) out[0] = m;
    return;
  }
  double s = 0.0;
  for (int i = threadIdx.x; i < P; i += 256) s += part[i];
  s = block_sum<256>(s, dl);
  if (threadIdx.x == 0) out[0] = kind == 1 ? (float)(s / (double)n) : (float)s;
}

// Rank-2 transpose (PERMUTE [1,0] materialized): 32x32 tiles staged through LDS (padded pitch)
// so both the read of X and the write of Y are coalesced.
__global__ void __launch_bounds__(256) transpose_kernel(const float* __restrict__ x,
                                                        float* __restrict__ y, int64_t R,
                                                        int64_t C) {
  __shared__ float tile[32][33];
  const int64_t r0 = (int64_t)blockIdx.y * 32, c0 = (int64_t)blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int k = ty; k < 32; k += 8) {
    const int64_t r = r0 + k, c = c0 + tx;
    if (r < R && c < C) tile[k][tx] = x[r * C + c];
  }
  __syncthreads();
  for (int k = ty; k < 32; k += 8) {
    const int64_t c = c0 + k, r = r0 + tx;
    if (r < R && c < C) y[c * R + r] = tile[tx][k];
  }
}

unsigned grid_for(int64_t n, int per_thread, int nt = 256) {
  int64_t g = (n + (int64_t)nt * per_thread - 1) / ((int64_t)nt * per_thread);
  if (g < 1) g = 1;
  if (g > 65536) g = 65536;
  return (unsigned)g;
}

}  // namespace

namespace {
// Recognizes a single-op chain: LOAD x -> rx [, LOAD y -> ry], OP (operands among rx, ry) -> rd,
// STORE rd -> out[o], every operand full-shape and 16-byte aligned. Fills the operand order the
// op reads (a, b) and returns the op, or -1.
int pw_single_op(const PwParams& p, const float** a, const float** b, float** out, bool* binary) {
  auto aligned = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; };
  const int n = p.n_instr;
  if (n != 3 && n != 4) return -1;
  const int nl = n - 2;
  int reg[2];
  const float* src[2];
  for (int i = 0; i < nl; ++i) {
    const PwInstr& l = p.code[i];
    if (l.op != PW_LOAD) return -1;
    const int k = l.a % PW_MAX_INPUTS;
    if (p.in[k] == nullptr || p.in_mode[k] != 0 || !aligned(p.in[k])) return -1;
    reg[i] = l.dst & (PW_REGS - 1);
    src[i] = p.in[k];
  }
  if (nl == 2 && reg[0] == reg[1]) return -1;
  const PwInstr& op = p.code[nl];
  const PwInstr& st = p.code[nl + 1];
  if (st.op != PW_STORE || (st.a & (PW_REGS - 1)) != (op.dst & (PW_REGS - 1))) return -1;
  float* o = p.out[st.dst & 1];
  if (o == nullptr || !aligned(o)) return -1;
  auto which = [&](int r) -> const float* {
    for (int i = 0; i < nl; ++i)
      if (reg[i] == (r & (PW_REGS - 1))) return src[i];
    return nullptr;
  };
  const bool bin = op.op == PW_ADD || op.op == PW_SUB || op.op == PW_MUL || op.op == PW_DIV ||
                   op.op == PW_MAX || op.op == PW_GT || op.op == PW_RELU_GRAD ||
                   op.op == PW_TANH_GRAD || op.op == PW_SIGMOID_GRAD;
  const bool un = op.op == PW_NEG || op.op == PW_RELU || op.op == PW_TANH ||
                  op.op == PW_SIGMOID || op.op == PW_EXP || op.op == PW_LOG || op.op == PW_SQRT;
  if (!bin && !un) return -1;
  *a = which(op.a);
  *b = bin ? which(op.b) : *a;
  if (*a == nullptr || *b == nullptr) return -1;
  *out = o;
  *binary = bin;
  return op.op;
}

template <int OP>
void launch_single(const float* a, const float* b, float* out, int64_t n, bool bin, hipStream_t s) {
  const unsigned g = grid_for(n, 8);
  if (bin) hipLaunchKernelGGL((pw_single_kernel<OP, true>), dim3(g), dim3(256), 0, s, a, b, out, n);
  else hipLaunchKernelGGL((pw_single_kernel<OP, false>), dim3(g), dim3(256), 0, s, a, b, out, n);
}
}  // namespace

hipError_t launch_pointwise(const PwParams& p, hipStream_t s) {
  const int64_t n = p.R * p.C;
  if (n <= 0) return hipSuccess;
  const float *a, *b;
  float* out;
  bool bin;
  switch (pw_single_op(p, &a, &b, &out, &bin)) {
    case PW_ADD: launch_single<PW_ADD>(a, b, out, n, bin, s); break;
    case PW_SUB: launch_single<PW_SUB>(a, b, out, n, bin, s); break;
    case PW_MUL: launch_single<PW_MUL>(a, b, out, n, bin, s); break;
    case PW_DIV: launch_single<PW_DIV>(a, b, out, n, bin, s); break;
    case PW_MAX: launch_single<PW_MAX>(a, b, out, n, bin, s); break;
    case PW_GT: launch_single<PW_GT>(a, b, out, n, bin, s); break;
    case PW_RELU_GRAD: launch_single<PW_RELU_GRAD>(a, b, out, n, bin, s); break;
    case PW_TANH_GRAD: launch_single<PW_TANH_GRAD>(a, b, out, n, bin, s); break;
    case PW_SIGMOID_GRAD: launch_single<PW_SIGMOID_GRAD>(a, b, out, n, bin, s); break;
    case PW_NEG: launch_single<PW_NEG>(a, b, out, n, bin, s); break;
    case PW_RELU: launch_single<PW_RELU>(a, b, out, n, bin, s); break;
    case PW_TANH: launch_single<PW_TANH>(a, b, out, n, bin, s); break;
    case PW_SIGMOID: launch_single<PW_SIGMOID>(a, b, out, n, bin, s); break;
    case PW_EXP: launch_single<PW_EXP>(a, b, out, n, bin, s); break;
    case PW_LOG: launch_single<PW_LOG>(a, b, out, n, bin, s); break;
    case PW_SQRT: launch_single<PW_SQRT>(a, b, out, n, bin, s); break;
    default:
      hipLaunchKernelGGL(pointwise_kernel, dim3(grid_for(n, 4)), dim3(PW_NT), 0, s, p);
  }
  return hipGetLastError();
}

hipError_t launch_transpose(const float* x, float* y, int64_t R, int64_t C, hipStream_t s) {
  if (R <= 0 || C <= 0) return hipSuccess;
  dim3 g((unsigned)((C + 31) / 32), (unsigned)((R + 31) / 32));
  hipLaunchKernelGGL(transpose_kernel, g, dim3(256), 0, s, x, y, R, C);
  return hipGetLastError();
}

hipError_t launch_fill(float* x, int64_t n, float value, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(fill_kernel, dim3(grid_for(n, 4)), dim3(256), 0, s, x, n, value);
  return hipGetLastError();
}
hipError_t launch_fill_u32(uint32_t* x, int64_t n, uint32_t value, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(fill_u32_kernel, dim3(grid_for(n, 4)), dim3(256), 0, s, x, n, value);
  return hipGetLastError();
}
hipError_t launch_copy(const float* src, float* dst, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  const bool aligned =
      ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15u) == 0;
  const int64_t n4 = aligned ? n / 4 : 0;
  if (n4 > 0) {
    const int64_t blocks = (n4 + 255) / 256;
    if (blocks > INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(copy_vec_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                       reinterpret_cast<const float4*>(src), reinterpret_cast<float4*>(dst), n4);
  }
  const int64_t rest = n - 4 * n4;
  if (rest > 0)
    hipLaunchKernelGGL(copy_kernel, dim3(grid_for(rest, 4)), dim3(256), 0, s, src + 4 * n4,
                       dst + 4 * n4, rest);
  return hipGetLastError();
}

int64_t colsum_partial_doubles(int64_t R, int64_t N) {
  if (R <= 0 || N <= 0) return 0;
  const int64_t rows = colsum_rows_per_panel(R, N);
  return ((R + rows - 1) / rows) * N;
}
hipError_t launch_colsum(const float* x, float* out, int64_t R, int64_t N, int64_t ldx,
                         double divisor, int accumulate, double* partial, hipStream_t s) {
  if (N <= 0) return hipSuccess;
  if (N <= CS_SMALL_MAX_N && R <= CS_SMALL_MAX_R) {
    hipLaunchKernelGGL(colsum_small, dim3((unsigned)((N + CS_COLS - 1) / CS_COLS)), dim3(1024), 0,
                       s, x, out, R, N, ldx, divisor, accumulate);
    return hipGetLastError();
  }
  const int64_t rows = colsum_rows_per_panel(R, N);
  const int64_t P = (R + rows - 1) / rows;
  if (P > 0) {
    if (N % 4 == 0 && ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0) {
      dim3 g1((unsigned)((N + 4 * CS_COLS - 1) / (4 * CS_COLS)), (unsigned)P);
      hipLaunchKernelGGL(colsum_pass1_v4, g1, dim3(256), 0, s, x, partial, R, N, ldx, rows);
    } else {
      dim3 g1((unsigned)((N + CS_COLS - 1) / CS_COLS), (unsigned)P);
      hipLaunchKernelGGL(colsum_pass1, g1, dim3(256), 0, s, x, partial, R, N, ldx, rows);
    }
  }
  hipLaunchKernelGGL(colsum_pass2, dim3((unsigned)((N + CS_COLS - 1) / CS_COLS)), dim3(256), 0, s,
                     partial, out, P, N, divisor, accumulate);
  return hipGetLastError();
}

hipError_t launch_colsum_finish(const double* partial, float* out, int64_t P, int64_t N,
                                hipStream_t s) {
  if (N <= 0) return hipSuccess;
  hipLaunchKernelGGL(colsum_pass2, dim3((unsigned)((N + CS_COLS - 1) / CS_COLS)), dim3(256), 0, s,
                     partial, out, P, N, 1.0, 0);
  return hipGetLastError();
}

hipError_t launch_row_reduce(const float* x, float* out, int64_t R, int64_t C, int kind,
                             hipStream_t s) {
  if (R <= 0) return hipSuccess;
  hipLaunchKernelGGL(row_reduce_kernel<256>, dim3((unsigned)R), dim3(256), 0, s, x, out, C, kind);
  return hipGetLastError();
}

int64_t reduce_all_partial_doubles(int64_t) { return RA_BLOCKS; }
hipError_t launch_reduce_all(const float* x, float* out, int64_t n, int kind, double* partial,
                             hipStream_t s) {
  const unsigned g = (unsigned)std::min<int64_t>(RA_BLOCKS, std::max<int64_t>(1, (n + 1023) / 1024));
  hipLaunchKernelGGL(reduce_all_pass1, dim3(g), dim3(256), 0, s, x, n, kind, partial);
  hipLaunchKernelGGL(reduce_all_pass2, dim3(1), dim3(256), 0, s, (const double*)partial, (int)g, n,
                     kind, out);
  return hipGetLastError();
}

}  // namespace shk
