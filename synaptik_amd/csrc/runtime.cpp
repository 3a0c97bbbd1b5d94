// C-ABI runtime of libsynaptik_hip.so: contexts, device buffers and op-list programs.
//
// Shape follows the reference's Metal native bridge (synaptik_metal_foundation.m:1681-1770 for
// context/buffers, :8573 and :9984-10083 for executable create/run): int32 status codes, opaque
// handles, out-pointers cleared on entry, no exception crosses the ABI.
//
// A program is decoded and validated once at create time (every step's operand extents are
// checked against its slots' byte sizes, so no launch can address outside a bound buffer),
// allocates one device arena for internal slots and reduction scratch, and is then run any
// number of times with caller-bound input/output buffers (inputs of kind INOUT are parameters and
// optimizer slots that the program updates in place).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <map>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <condition_variable>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/synaptik_hip.h"
#include "kernels.h"

// Device memory of shk_hip_program_run_static, the entry point that allocates nothing: a run's
// status word, reduction scratch and internal slots, laid out as a lease arena. Each device the
// library runs on holds one copy of it until the process ends. Host code never uses this name
// as an address (on the host it names a stand-in): the device address of each device's copy is
// resolved once, at context creation, and kept in g_scratch_address.
constexpr uint64_t kStaticScratchBytes = 64ull << 20;
__device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

namespace {

thread_local std::string g_last_error;

int32_t fail(int32_t status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return status;
}

#define HIP_TRY(expr)                                                                         \
  do {                                                                                        \
    hipError_t e_ = (expr);                                                                   \
    if (e_ != hipSuccess)                                                                     \
      return fail(SHK_HIP_STATUS_DEVICE_ERROR, "%s failed: %s", #expr, hipGetErrorName(e_));  \
  } while (0)

// Per device ordinal: the device address of `scratch` (null until resolved), and whether its
// resolution was attempted; guarded by g_scratch_mutex.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_address[kMaxDevices] = {};
hipError_t g_scratch_error[kMaxDevices] = {};
// One run at a time per device uses that device's copy of `scratch`: held by
// shk_hip_program_run_static from the arena clear until its stream has drained, whichever
// context the run goes through.
std::mutex g_static_run_mutex[kMaxDevices];

// Resolves this device's copy of `scratch` (the device current; once per device).
void resolve_static_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) return;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_address[device] != nullptr) return;
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e == hipSuccess && ptr != nullptr) {
    g_scratch_address[device] = ptr;
  } else {
    g_scratch_error[device] = e != hipSuccess ? e : hipErrorInvalidSymbol;
    (void)hipGetLastError();
  }
}

constexpr uint32_t kContextMagic = 0x43484B53u;  // "SKHC"
constexpr uint32_t kBufferMagic = 0x42484B53u;
constexpr uint32_t kProgramMagic = 0x50484B53u;
constexpr uint32_t kImageMagic = 0x504B4853u;    // "SHKP" little-endian
constexpr uint32_t kImageVersion = 1u;

// A context stays alive while any buffer or program created from it is alive: the owner's
// release drops one reference, every child holds one, and the last release destroys it. A child
// released after its owner therefore never touches freed memory.
struct Context {
  uint32_t magic = kContextMagic;
  int device = 0;
  hipStream_t stream = nullptr;
  // pinned status word of shk_hip_program_run_static runs, which hold the context mutex for
  // their whole duration
  uint32_t* host_status = nullptr;
  // Device staging of canonical publications: a 256-byte status block, then the packed bytes.
  // Grown on demand, guarded by `mutex`, freed with the context.
  uint8_t* pub_staging = nullptr;
  uint64_t pub_staging_bytes = 0;
  // Staged uploads (shk_hip_buffer_upload_staged): a second stream at the default priority and a
  // ring of pinned host chunks, created on first use, freed with the context.
  hipStream_t copy_stream = nullptr;
  // Second compute stream (default priority) for the steps a program schedules beside the main
  // chain; created with the first program that uses it.
  hipStream_t side_stream = nullptr;
  uint8_t* ring[4] = {nullptr, nullptr, nullptr, nullptr};
  hipEvent_t ring_free[4] = {nullptr, nullptr, nullptr, nullptr};
  bool ring_used[4] = {false, false, false, false};
  int ring_next = 0;
  std::mutex mutex;
  std::atomic<int64_t> refs{1};
  std::atomic<bool> released{false};
};

void context_unref(Context* c) {
  if (c->refs.fetch_sub(1) != 1) return;
  (void)hipSetDevice(c->device);
  if (c->copy_stream != nullptr) {
    (void)hipStreamSynchronize(c->copy_stream);
    (void)hipStreamDestroy(c->copy_stream);
  }
  for (int i = 0; i < 4; ++i) {
    if (c->ring_free[i] != nullptr) (void)hipEventDestroy(c->ring_free[i]);
    if (c->ring[i] != nullptr) (void)hipHostFree(c->ring[i]);
  }
  if (c->side_stream != nullptr) {
    (void)hipStreamSynchronize(c->side_stream);
    (void)hipStreamDestroy(c->side_stream);
  }
  (void)hipStreamSynchronize(c->stream);
  (void)hipStreamDestroy(c->stream);
  (void)hipHostFree(c->host_status);
  if (c->pub_staging != nullptr) (void)hipFree(c->pub_staging);
  c->magic = 0;
  delete c;
}

struct Buffer {
  uint32_t magic = kBufferMagic;
  Context* ctx = nullptr;
  void* ptr = nullptr;
  uint64_t bytes = 0;
  bool owned = true;
  // Cross-stream ordering (guarded by ctx->mutex): a staged upload into this buffer still in
  // flight on the copy stream (upload_done), and the end of the last asynchronous run that bound
  // it on the compute stream (last_use). Created on first use.
  hipEvent_t upload_done = nullptr;
  bool upload_pending = false;
  hipEvent_t last_use = nullptr;
  bool use_pending = false;
};

// Orders `stream` after a staged upload into b that may still be in flight (caller holds the
// context mutex).
hipError_t order_after_upload(Buffer* b, hipStream_t stream) {
  if (!b->upload_pending) return hipSuccess;
  const hipError_t e = hipStreamWaitEvent(stream, b->upload_done, 0);
  if (e == hipSuccess && stream == b->ctx->stream) b->upload_pending = false;
  return e;
}

enum SlotKind : uint32_t { SLOT_INTERNAL = 0, SLOT_INPUT = 1, SLOT_OUTPUT = 2, SLOT_INOUT = 3 };
enum DType : uint32_t { DT_F32 = 0, DT_I32 = 1, DT_I64 = 2, DT_U8 = 3, DT_F64 = 4 };

enum Opcode : uint32_t {
  OP_GEMM = 1,
  OP_COLSUM = 2,
  OP_ROW_REDUCE = 3,
  OP_REDUCE_ALL = 4,
  OP_POINTWISE = 5,
  OP_SOFTMAX = 6,
  OP_SOFTMAX_BWD = 7,
  OP_LSE_BWD = 8,
  OP_MSE = 9,
  OP_CE_INDEX = 10,
  OP_OPTIMIZER = 11,
  OP_STEP_COMMIT = 12,
  OP_FILL = 13,
  OP_COPY = 14,
  OP_TRANSPOSE = 15,
  OP_CE_HEAD = 16,
};

#pragma pack(push, 1)
struct ImageHeader {
  uint32_t magic, version, n_slots, n_steps;
};
struct SlotRecord {
  uint64_t bytes;
  uint32_t kind, ext_index, dtype, flags;
};
struct StepRecord {
  uint32_t opcode, payload_bytes;
  int32_t slot[8];
  int64_t iarg[16];
  float farg[8];
};
struct OptEntry {
  int32_t p, g, m, v;
  int32_t pn, mn, vn, pad;
  int64_t n;
};
#pragma pack(pop)
static_assert(sizeof(SlotRecord) == 24, "slot record layout");
static_assert(sizeof(StepRecord) == 200, "step record layout");
static_assert(sizeof(OptEntry) == 40, "optimizer entry layout");
static_assert(sizeof(shk::PwInstr) == 12, "pointwise instruction layout");

struct Step {
  StepRecord rec;
  std::vector<uint8_t> payload;
};

// Per-run state of a program (the analogue of the reference's RunState-owned buffers and
// workspaces, docs/backend-guide/writing-a-backend.md:140-142): a device arena holding the
// status word, the reduction scratch of each stream and the internal slots, a pinned host word
// the run's status is published to, the events of one run, and the HIP graphs captured over this
// arena. A run holds one lease from acquisition until its completion is observed; concurrent runs
// of one program hold different leases, so nothing one run writes is visible to another.
struct Lease {
  void* arena = nullptr;
  uint32_t* status = nullptr;      // device status word (first bytes of the arena)
  double* scratch = nullptr;       // reduction partials of the context stream's steps
  double* scratch_side = nullptr;  // ... of the side stream's steps (two-stream plan)
  uint32_t* host_status = nullptr; // pinned; written by the run's status publication kernel
  hipEvent_t done = nullptr;       // end of the run
  // Private streams the lease's graphs are captured on (then launched on the context stream):
  // another thread may synchronize the shared streams at any time, which would invalidate a
  // capture running on them.
  hipStream_t cap0 = nullptr, cap1 = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  std::vector<hipEvent_t> step_done;  // per step the other stream waits for
  std::vector<hipEvent_t> events;     // per-step timing (profiled runs), created on first use
  // HIP-graph replay: the step sequence captured once per distinct set of bound pointers and
  // schedule (up to 8 cached, oldest evicted)
  std::map<std::vector<void*>, hipGraphExec_t> graph_cache;
  std::vector<std::vector<void*>> graph_order;
  bool graphs_ok = true;  // a capture failed on this lease: launch step by step from then on
  // Every run ends with a kernel that copies the status word to host_status and clears it, so
  // the next run on this lease starts from a clear word. Until a run has completed that way (a
  // new lease, a failed launch or execution) the next run clears the word first.
  bool status_clear = false;
};

struct Program {
  uint32_t magic = kProgramMagic;
  Context* ctx = nullptr;
  // ---- immutable after create: shared by every run ----
  std::vector<SlotRecord> slots;
  std::vector<Step> steps;
  uint32_t n_inputs = 0, n_outputs = 0;
  uint64_t arena_bytes = 0;               // per lease
  uint64_t scratch_off = 0, scratch_side_off = 0;
  std::vector<uint64_t> internal_offset;  // per slot (internal only), within a lease's arena
  // Two-stream schedule (plan_streams): step j runs on the context stream (0) or its side
  // stream (1), first waiting for the events recorded after the steps in wait_for[j];
  // record_after[j] marks steps other-stream steps depend on. side_steps == 0: one stream.
  uint32_t side_steps = 0;
  std::vector<uint8_t> stream_of, record_after;
  std::vector<std::vector<uint32_t>> wait_for;
  // Trailing steps that no later launched step depends on, performed by the run's last launch
  // (the publication kernel) in unprofiled runs instead of launches of their own (-1: none): a
  // classifier-loss MEAN (OP_CE_HEAD finish) and a small staged optimizer pass.
  int64_t folded_finish = -1;
  int64_t folded_opt = -1;
  bool folded(size_t j) const {
    return (int64_t)j == folded_finish || (int64_t)j == folded_opt;
  }
  // ---- settings and the lease pool, guarded by `mutex` ----
  std::mutex mutex;
  std::condition_variable lease_freed;
  bool graphs = true;
  bool concurrent = false;  // the two-stream plan is active
  bool profiling = false;
  uint64_t profiled_runs = 0;
  std::vector<double> step_ms;
  std::vector<Lease*> leases;  // every lease, in creation order
  std::vector<Lease*> idle;    // leases no run holds
  uint32_t max_leases = 4;
  // Asynchronous runs (shk_hip_program_run_async) not yet waited for, oldest first; each keeps
  // its lease until shk_hip_program_wait (or the program's next run) observes its completion.
  std::vector<Lease*> pending;
};

template <typename T, uint32_t M>
T* checked(void* h) {
  if (h == nullptr) return nullptr;
  T* t = static_cast<T*>(h);
  return t->magic == M ? t : nullptr;
}

// A context handle the owner has not released yet.
Context* live_context(void* h) {
  Context* c = checked<Context, kContextMagic>(h);
  return (c != nullptr && !c->released.load()) ? c : nullptr;
}

uint64_t dtype_size(uint32_t dt) {
  switch (dt) {
    case DT_F32: case DT_I32: return 4;
    case DT_I64: case DT_F64: return 8;
    case DT_U8: return 1;
    default: return 0;
  }
}

// ---- create-time validation helpers ----
struct Validator {
  const std::vector<SlotRecord>& slots;
  size_t step;
  int32_t err = SHK_HIP_STATUS_OK;

  bool slot_ok(int32_t s, bool optional, const char* role) {
    if (s < 0) {
      if (optional) return true;
      err = fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "step %zu: missing %s slot", step, role);
      return false;
    }
    if ((size_t)s >= slots.size()) {
      err = fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "step %zu: %s slot %d out of range",
                 step, role, s);
      return false;
    }
    return true;
  }
  // Requires that slot s holds at least `elems` elements of dtype dt.
  bool holds(int32_t s, int64_t elems, uint32_t dt, const char* role) {
    if (s < 0) return true;
    uint64_t need;
    if (elems < 0 || __builtin_mul_overflow((uint64_t)elems, dtype_size(dt), &need)) {
      err = fail(SHK_HIP_STATUS_UNSUPPORTED_SHAPE, "step %zu: extent of %s is negative or too large",
                 step, role);
      return false;
    }
    if (slots[s].dtype != dt) {
      err = fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "step %zu: %s slot %d has dtype %u, expected %u",
                 step, role, s, slots[s].dtype, dt);
      return false;
    }
    if (slots[s].bytes < need) {
      err = fail(SHK_HIP_STATUS_RANGE_OUT_OF_BOUNDS,
                 "step %zu: %s slot %d has %llu bytes, operand needs %llu", step, role, s,
                 (unsigned long long)slots[s].bytes, (unsigned long long)need);
      return false;
    }
    return true;
  }
  bool writable(int32_t s, const char* role) {
    if (s < 0) return true;
    if (slots[s].kind == SLOT_INPUT) {
      err = fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "step %zu: %s writes read-only input slot %d",
                 step, role, s);
      return false;
    }
    return true;
  }
};

// Product of two extents, or -1 when either is negative or the product does not fit int64
// (every extent product of an image goes through here: the image is untrusted input).
int64_t prod(int64_t a, int64_t b) {
  int64_t r;
  if (a < 0 || b < 0 || __builtin_mul_overflow(a, b, &r)) return -1;
  return r;
}

// Extent (in elements) spanned by a row-major matrix view of `rows` x `cols` with leading dim ld,
// or -1 when it does not fit int64.
int64_t span(int64_t rows, int64_t cols, int64_t ld) {
  if (rows <= 0 || cols <= 0) return 0;
  int64_t r;
  if (ld < 0 || __builtin_mul_overflow(rows - 1, ld, &r) || __builtin_add_overflow(r, cols, &r))
    return -1;
  return r;
}

// GEMM whose epilogue stages an optimizer update from the gradient it computes (payload: one
// tensor-table entry p, m, v, pn, mn, vn over the [M, N] result; slot 6: step counter). The
// gradient itself is not stored, so C, bias, aux, column sum, activation and accumulation are
// absent. Shapes and leading dimensions were checked by the caller.
int32_t validate_gemm_update(Validator& v, size_t idx, const Step& st) {
  const StepRecord& r = st.rec;
  const int32_t* s = r.slot;
  const int64_t* a = r.iarg;
  const int64_t M = a[0], N = a[1], K = a[2], lda = a[3], ldb = a[4], ldc = a[5];
  const int64_t tA = a[7], tB = a[8], kind = a[12];
  if (st.payload.size() != sizeof(OptEntry))
    return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "step %zu: fused update needs one tensor entry", idx);
  if (s[2] >= 0 || s[3] >= 0 || s[4] >= 0 || s[5] >= 0 || a[9] != 0 || a[10] != 0 || a[11] != 0 ||
      ldc != N || kind < 0 || kind > 2)
    return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED,
                "step %zu: fused update GEMM takes no C, bias, aux, column sum, activation or accumulation", idx);
  const OptEntry& e = *reinterpret_cast<const OptEntry*>(st.payload.data());
  const bool adam = kind != 0;
  if (e.n != M * N || e.g >= 0)
    return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "step %zu: fused update entry does not cover the result", idx);
  if ((e.m >= 0) != (e.mn >= 0) || (e.v >= 0) != (e.vn >= 0))
    return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "step %zu: staged update lacks a candidate buffer", idx);
  if (!v.slot_ok(s[0], false, "A") || !v.slot_ok(s[1], false, "B") ||
      !v.slot_ok(s[6], false, "step counter") || !v.holds(s[6], 1, DT_I64, "step counter") ||
      !v.holds(s[0], K == 0 ? 0 : (tA ? span(K, M, lda) : span(M, K, lda)), DT_F32, "A") ||
      !v.holds(s[1], K == 0 ? 0 : (tB ? span(N, K, ldb) : span(K, N, ldb)), DT_F32, "B"))
    return v.err;
  if (!v.slot_ok(e.p, false, "param") || !v.slot_ok(e.m, !adam, "momentum") ||
      !v.slot_ok(e.v, !adam, "second moment") || !v.slot_ok(e.pn, false, "param candidate") ||
      !v.slot_ok(e.mn, true, "momentum candidate") || !v.slot_ok(e.vn, true, "second moment candidate") ||
      !v.holds(e.p, e.n, DT_F32, "param") || !v.holds(e.m, e.n, DT_F32, "momentum") ||
      !v.holds(e.v, e.n, DT_F32, "second moment") || !v.holds(e.pn, e.n, DT_F32, "param candidate") ||
      !v.holds(e.mn, e.n, DT_F32, "momentum candidate") ||
      !v.holds(e.vn, e.n, DT_F32, "second moment candidate") ||
      !v.writable(e.pn, "param candidate") || !v.writable(e.mn, "momentum candidate") ||
      !v.writable(e.vn, "second moment candidate"))
    return v.err;
  return SHK_HIP_STATUS_OK;
}

int32_t validate_step(const std::vector<SlotRecord>& slots, size_t idx, const Step& st,
                      uint64_t* scratch_doubles) {
  Validator v{slots, idx};
  const StepRecord& r = st.rec;
  const int32_t* s = r.slot;
  const int64_t* a = r.iarg;
  auto need = [&](uint64_t d) { *scratch_doubles = std::max<uint64_t>(*scratch_doubles, d); };
  switch (r.opcode) {
    case OP_GEMM: {
      const int64_t M = a[0], N = a[1], K = a[2], lda = a[3], ldb = a[4], ldc = a[5], ldaux = a[6];
      const int64_t tA = a[7], tB = a[8], act = a[9], mode = a[10];
      if (M < 0 || N < 0 || K < 0 || (tA != 0 && tA != 1) || (tB != 0 && tB != 1) || act < 0 ||
          act > 3 || mode < 0 || mode > 2)
        return fail(SHK_HIP_STATUS_UNSUPPORTED_SHAPE, "step %zu: invalid GEMM attributes", idx);
      if (M > INT32_MAX / 2 || N > INT32_MAX / 2 || K > INT32_MAX)
        return fail(SHK_HIP_STATUS_UNSUPPORTED_SHAPE, "step %zu: GEMM extent too large", idx);
      const bool empty = M == 0 || N == 0;  // touches no memory
      if (!empty && ((K > 0 && (tA ? lda < std::max<int64_t>(M, 1) : lda < K)) ||
          (K > 0 && (tB ? ldb < K : ldb < std::max<int64_t>(N, 1))) ||
          ldc < std::max<int64_t>(N, 1) || (mode != 0 && ldaux < std::max<int64_t>(N, 1))))
        return fail(SHK_HIP_STATUS_UNSUPPORTED_SHAPE, "step %zu: GEMM leading dimension too small", idx);
      if (mode == 1 && s[4] < 0)
        return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "step %zu: activation gradient needs aux", idx);
      if (mode == 2) {
        // forward with its cotangent: dY in aux, dZ in slot 7, no accumulation or update, and
        // dZ distinct from every slot the step reads or writes
        if (s[4] < 0 || s[7] < 0 || a[11] != 0 || !st.payload.empty())
          return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED,
                      "step %zu: a forward GEMM with its cotangent needs dY and dZ slots", idx);
        if (!v.slot_ok(s[7], false, "dZ") || !v.holds(s[7], span(M, N, ldaux), DT_F32, "dZ") ||
            !v.writable(s[7], "dZ"))
          return v.err;
        for (int k = 0; k < 6; ++k)
          if (s[k] == s[7])
            return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "step %zu: dZ aliases another operand", idx);
        if (s[4] == s[2])  // the epilogue stores C before it reads dY
          return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "step %zu: dY aliases C", idx);
      } else if (s[7] >= 0) {
        return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "step %zu: dZ slot without mode 2", idx);
      }
      if (!st.payload.empty()) {
        const int32_t u = validate_gemm_update(v, idx, st);
        if (u == SHK_HIP_STATUS_OK)
          need((uint64_t)((shk::gemm_workspace_floats(M, N, K, false) + 1) / 2));  // in doubles
        return u;
      }
      if (!v.slot_ok(s[0], false, "A") || !v.slot_ok(s[1], false, "B") || !v.slot_ok(s[2], false, "C") ||
          !v.slot_ok(s[3], true, "bias") || !v.slot_ok(s[4], true, "aux"))
        return v.err;
      if (!v.holds(s[0], K == 0 ? 0 : (tA ? span(K, M, lda) : span(M, K, lda)), DT_F32, "A") ||
          !v.holds(s[1], K == 0 ? 0 : (tB ? span(N, K, ldb) : span(K, N, ldb)), DT_F32, "B") ||
          !v.holds(s[2], span(M, N, ldc), DT_F32, "C") || !v.holds(s[3], N, DT_F32, "bias") ||
          !v.holds(s[4], span(M, N, ldaux), DT_F32, "aux") || !v.writable(s[2], "C"))
        return v.err;
      if (!v.slot_ok(s[5], true, "column sum") || !v.holds(s[5], N, DT_F32, "column sum") ||
          !v.writable(s[5], "column sum"))
        return v.err;
      need((uint64_t)((shk::gemm_workspace_floats(M, N, K, s[5] >= 0) + 1) / 2));  // in doubles
      // the separate column-sum pass of a split GEMM reuses the workspace for its partials
      if (s[5] >= 0) need((uint64_t)shk::colsum_partial_doubles(M, N));
      return SHK_HIP_STATUS_OK;
    }
    case OP_COLSUM: {
      const int64_t R = a[0], N = a[1], ldx = a[2];
      if (R < 0 || N < 0 || ldx < std::max<int64_t>(N, 1))
        return fail(SHK_HIP_STATUS_UNSUPPORTED_SHAPE, "step %zu: invalid COLSUM shape", idx);
      if (!v.slot_ok(s[0], false, "X") || !v.slot_ok(s[1], false, "out") ||
          !v.holds(s[0], span(R, N, ldx), DT_F32, "X") || !v.holds(s[1], N, DT_F32, "out") ||
          !v.writable(s[1], "out"))
        return v.err;
      need((uint64_t)shk::colsum_partial_doubles(R, N));
      return SHK_HIP_STATUS_OK;
    }
    case OP_ROW_REDUCE: {
      const int64_t R = a[0], C = a[1], kind = a[2];
      if (R < 0 || C < 0 || kind < 0 || kind > 3 || R > INT32_MAX)
        return fail(SHK_HIP_STATUS_UNSUPPORTED_SHAPE, "step %zu: invalid row reduction", idx);
      if (!v.slot_ok(s[0], false, "X") || !v.slot_ok(s[1], false, "out") ||
          !v.holds(s[0], prod(R, C), DT_F32, "X") || !v.holds(s[1], R, DT_F32, "out") ||
          !v.writable(s[1], "out"))
        return v.err;
      return SHK_HIP_STATUS_OK;
    }
    case OP_REDUCE_ALL: {
      const int64_t n = a[0], kind = a[1];
      if (n < 0 || kind < 0 || kind > 2)
        return fail(SHK_HIP_STATUS_UNSUPPORTED_SHAPE, "step %zu: invalid reduction", idx);
      if (!v.slot_ok(s[0], false, "X") || !v.slot_ok(s[1], false, "out") ||
          !v.holds(s[0], n, DT_F32, "X") || !v.holds(s[1], 1, DT_F32, "out") ||
          !v.writable(s[1], "out"))
        return v.err;
      need((uint64_t)shk::reduce_all_partial_doubles(n));
      return SHK_HIP_STATUS_OK;
    }
    case OP_POINTWISE: {
      const int64_t R = a[0], C = a[1];
      if (R < 0 || C < 0) return fail(SHK_HIP_STATUS_UNSUPPORTED_SHAPE, "step %zu: invalid pointwise shape", idx);
      const size_t n_instr = st.payload.size() / sizeof(shk::PwInstr);
      if (st.payload.size() % sizeof(shk::PwInstr) != 0 || n_instr == 0 ||
          n_instr > (size_t)shk::PW_MAX_INSTR)
        return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "step %zu: bad pointwise program", idx);
      for (int k = 0; k < shk::PW_MAX_INPUTS; ++k) {
        if (!v.slot_ok(s[k], true, "pointwise input")) return v.err;
        const int64_t mode = a[2 + k];
        const int64_t ext = mode == 0 ? prod(R, C) : mode == 1 ? C : mode == 2 ? R : 1;
        if (mode < 0 || mode > 3)
          return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "step %zu: bad broadcast mode", idx);
        if (!v.holds(s[k], ext, DT_F32, "pointwise input")) return v.err;
      }
      for (int o = 0; o < shk::PW_MAX_OUTPUTS; ++o) {
        if (!v.slot_ok(s[6 + o], true, "pointwise output") || !v.holds(s[6 + o], prod(R, C), DT_F32, "pointwise output") ||
            !v.writable(s[6 + o], "pointwise output"))
          return v.err;
      }
      const shk::PwInstr* code = reinterpret_cast<const shk::PwInstr*>(st.payload.data());
      for (size_t i = 0; i < n_instr; ++i) {
        const shk::PwInstr& in = code[i];
        if (in.op > 19 || in.dst >= 8 || in.a >= 8 || in.b >= 8 || in.c >= 8)
          return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "step %zu: bad pointwise instruction %zu", idx, i);
        if (in.op == 0 && (in.a >= shk::PW_MAX_INPUTS || s[in.a] < 0))
          return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "step %zu: load of unbound input %u", idx, in.a);
        if (in.op == 17 && (in.dst >= shk::PW_MAX_OUTPUTS || s[6 + in.dst] < 0))
          return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "step %zu: store to unbound output %u", idx, in.dst);
      }
      return SHK_HIP_STATUS_OK;
    }
    case OP_SOFTMAX: {
      const int64_t R = a[0], C = a[1];
      if (R < 0 || C < 0 || R > INT32_MAX)
        return fail(SHK_HIP_STATUS_UNSUPPORTED_SHAPE, "step %zu: invalid softmax shape", idx);
      if (!v.slot_ok(s[0], false, "X") || !v.slot_ok(s[1], false, "Y") || !v.slot_ok(s[2], true, "lse") ||
          !v.holds(s[0], prod(R, C), DT_F32, "X") || !v.holds(s[1], prod(R, C), DT_F32, "Y") ||
          !v.holds(s[2], R, DT_F32, "lse") || !v.writable(s[1], "Y") || !v.writable(s[2], "lse"))
        return v.err;
      return SHK_HIP_STATUS_OK;
    }
    case OP_SOFTMAX_BWD: {
      const int64_t R = a[0], C = a[1];
      if (R < 0 || C < 0 || R > INT32_MAX)
        return fail(SHK_HIP_STATUS_UNSUPPORTED_SHAPE, "step %zu: invalid softmax shape", idx);
      if (!v.slot_ok(s[0], false, "Y") || !v.slot_ok(s[1], false, "G") || !v.slot_ok(s[2], false, "dX") ||
          !v.slot_ok(s[3], true, "rowscale") || !v.holds(s[0], prod(R, C), DT_F32, "Y") ||
          !v.holds(s[1], prod(R, C), DT_F32, "G") || !v.holds(s[2], prod(R, C), DT_F32, "dX") ||
          !v.holds(s[3], R, DT_F32, "rowscale") || !v.writable(s[2], "dX"))
        return v.err;
      return SHK_HIP_STATUS_OK;
    }
    case OP_LSE_BWD: {
      const int64_t R = a[0], C = a[1];
      if (R < 0 || C < 0) return fail(SHK_HIP_STATUS_UNSUPPORTED_SHAPE, "step %zu: invalid LSE shape", idx);
      if (!v.slot_ok(s[0], false, "X") || !v.slot_ok(s[1], false, "lse") || !v.slot_ok(s[2], true, "g") ||
          !v.slot_ok(s[3], false, "dX") || !v.holds(s[0], prod(R, C), DT_F32, "X") ||
          !v.holds(s[1], R, DT_F32, "lse") || !v.holds(s[2], R, DT_F32, "g") ||
          !v.holds(s[3], prod(R, C), DT_F32, "dX") || !v.writable(s[3], "dX"))
        return v.err;
      return SHK_HIP_STATUS_OK;
    }
    case OP_MSE: {
      const int64_t n = a[0];
      if (n <= 0 || (a[1] != 0 && a[1] != 1))
        return fail(SHK_HIP_STATUS_UNSUPPORTED_SHAPE, "step %zu: invalid MSE", idx);
      if (!v.slot_ok(s[0], false, "P") || !v.slot_ok(s[1], false, "T") || !v.slot_ok(s[2], false, "loss") ||
          !v.slot_ok(s[3], true, "grad") || !v.holds(s[0], n, DT_F32, "P") || !v.holds(s[1], n, DT_F32, "T") ||
          !v.holds(s[2], 1, DT_F32, "loss") || !v.holds(s[3], n, DT_F32, "grad") ||
          !v.writable(s[2], "loss") || !v.writable(s[3], "grad"))
        return v.err;
      need((uint64_t)shk::mse_partial_doubles(n));
      return SHK_HIP_STATUS_OK;
    }
    case OP_CE_INDEX: {
      const int64_t R = a[0], C = a[1], is64 = a[2];
      if (R < 0 || C <= 0 || (is64 != 0 && is64 != 1))
        return fail(SHK_HIP_STATUS_UNSUPPORTED_SHAPE, "step %zu: invalid cross-entropy shape", idx);
      if (!v.slot_ok(s[0], false, "logits") || !v.slot_ok(s[1], false, "target") ||
          !v.slot_ok(s[2], false, "loss") || !v.slot_ok(s[3], true, "grad") ||
          !v.holds(s[0], prod(R, C), DT_F32, "logits") || !v.holds(s[1], R, is64 ? DT_I64 : DT_I32, "target") ||
          !v.holds(s[2], 1, DT_F32, "loss") || !v.holds(s[3], prod(R, C), DT_F32, "grad") ||
          !v.writable(s[2], "loss") || !v.writable(s[3], "grad"))
        return v.err;
      need((uint64_t)shk::index_ce_partial_doubles(R));
      return SHK_HIP_STATUS_OK;
    }
    case OP_CE_HEAD: {
      const int64_t R = a[0], K = a[1], J = a[2], act = a[3], phase = a[4], is64 = a[5];
      if (phase == 1) {
        if (R < 0) return fail(SHK_HIP_STATUS_UNSUPPORTED_SHAPE, "step %zu: invalid head loss", idx);
        if (!v.slot_ok(s[0], false, "row losses") || !v.slot_ok(s[1], false, "loss") ||
            !v.holds(s[0], R, DT_F32, "row losses") || !v.holds(s[1], 1, DT_F32, "loss") ||
            !v.writable(s[1], "loss"))
          return v.err;
        if (s[0] == s[1])
          return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "step %zu: head loss aliases its input", idx);
        return SHK_HIP_STATUS_OK;
      }
      if (phase != 0 || R < 0 || K <= 0 || J < 1 || J > 16 || act < 0 || act > 3 ||
          (is64 != 0 && is64 != 1))
        return fail(SHK_HIP_STATUS_UNSUPPORTED_SHAPE, "step %zu: invalid classifier head", idx);
      if (!v.slot_ok(s[0], false, "head input") || !v.slot_ok(s[1], false, "head weight") ||
          !v.slot_ok(s[2], true, "head bias") || !v.slot_ok(s[3], false, "target") ||
          !v.slot_ok(s[4], true, "logits") || !v.slot_ok(s[5], false, "logit cotangent") ||
          !v.slot_ok(s[6], true, "input cotangent") || !v.slot_ok(s[7], false, "row losses") ||
          !v.holds(s[0], prod(R, K), DT_F32, "head input") ||
          !v.holds(s[1], prod(J, K), DT_F32, "head weight") || !v.holds(s[2], J, DT_F32, "head bias") ||
          !v.holds(s[3], R, is64 ? DT_I64 : DT_I32, "target") ||
          !v.holds(s[4], prod(R, J), DT_F32, "logits") ||
          !v.holds(s[5], prod(R, J), DT_F32, "logit cotangent") ||
          !v.holds(s[6], prod(R, K), DT_F32, "input cotangent") ||
          !v.holds(s[7], R, DT_F32, "row losses") || !v.writable(s[4], "logits") ||
          !v.writable(s[5], "logit cotangent") || !v.writable(s[6], "input cotangent") ||
          !v.writable(s[7], "row losses"))
        return v.err;
      // the written slots are distinct from each other and from every slot the head reads
      for (int i = 4; i < 8; ++i) {
        if (s[i] < 0) continue;
        for (int k = 0; k < 8; ++k)
          if (k != i && s[k] == s[i])
            return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED,
                        "step %zu: classifier head slot %d is used twice", idx, s[i]);
      }
      return SHK_HIP_STATUS_OK;
    }
    case OP_OPTIMIZER: {
      const int64_t kind = a[0], phase = a[1];
      if (kind < 0 || kind > 5 || phase < 0 || phase > 2 || (phase == 2 && kind > 2))
        return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "step %zu: invalid optimizer", idx);
      if (!v.slot_ok(s[0], false, "step counter") || !v.holds(s[0], 1, DT_I64, "step counter"))
        return v.err;
      const size_t n = st.payload.size() / sizeof(OptEntry);
      if (st.payload.size() % sizeof(OptEntry) != 0 || n == 0 || n > (size_t)shk::OPT_MAX_TENSORS)
        return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "step %zu: bad optimizer tensor table", idx);
      const OptEntry* e = reinterpret_cast<const OptEntry*>(st.payload.data());
      for (size_t i = 0; i < n; ++i) {
        const bool adam = kind == 1 || kind == 2;
        const bool needs_m = adam || kind >= 3;  // accumulation kinds use m as the accumulator
        if (!v.slot_ok(e[i].p, false, "param") || !v.slot_ok(e[i].g, false, "grad") ||
            !v.slot_ok(e[i].m, !needs_m, "momentum") || !v.slot_ok(e[i].v, !adam, "second moment") ||
            !v.holds(e[i].p, e[i].n, DT_F32, "param") || !v.holds(e[i].g, e[i].n, DT_F32, "grad") ||
            !v.holds(e[i].m, e[i].n, DT_F32, "momentum") || !v.holds(e[i].v, e[i].n, DT_F32, "second moment"))
          return v.err;
        // writability follows what the step writes: phase 1 updates p,m,v in place; kind 3 writes
        // p; kinds 4 and 5 write m; phase 0 and phase 2 leave the current tensors untouched
        const bool in_place = (kind <= 2 && phase == 1);
        if ((in_place || kind == 3) && !v.writable(e[i].p, "param")) return v.err;
        if ((in_place || kind >= 4) && !v.writable(e[i].m, "momentum")) return v.err;
        if (in_place && !v.writable(e[i].v, "second moment")) return v.err;
        if (phase == 2) {
          // candidates must exist wherever a current tensor exists
          if ((e[i].m >= 0) != (e[i].mn >= 0) || (e[i].v >= 0) != (e[i].vn >= 0))
            return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "step %zu: staged update lacks a candidate buffer", idx);
          if (!v.slot_ok(e[i].pn, false, "param candidate") || !v.slot_ok(e[i].mn, true, "momentum candidate") ||
              !v.slot_ok(e[i].vn, true, "second moment candidate") ||
              !v.holds(e[i].pn, e[i].n, DT_F32, "param candidate") ||
              !v.holds(e[i].mn, e[i].n, DT_F32, "momentum candidate") ||
              !v.holds(e[i].vn, e[i].n, DT_F32, "second moment candidate") ||
              !v.writable(e[i].pn, "param candidate") || !v.writable(e[i].mn, "momentum candidate") ||
              !v.writable(e[i].vn, "second moment candidate"))
            return v.err;
        }
      }
      return SHK_HIP_STATUS_OK;
    }
    case OP_STEP_COMMIT:
      if (!v.slot_ok(s[0], false, "step counter") || !v.holds(s[0], 1, DT_I64, "step counter") ||
          !v.writable(s[0], "step counter"))
        return v.err;
      return SHK_HIP_STATUS_OK;
    case OP_FILL:
      if (a[0] < 0) return fail(SHK_HIP_STATUS_UNSUPPORTED_SHAPE, "step %zu: invalid fill", idx);
      if (!v.slot_ok(s[0], false, "X") || !v.holds(s[0], a[0], DT_F32, "X") || !v.writable(s[0], "X"))
        return v.err;
      return SHK_HIP_STATUS_OK;
    case OP_COPY:
      if (a[0] < 0) return fail(SHK_HIP_STATUS_UNSUPPORTED_SHAPE, "step %zu: invalid copy", idx);
      if (!v.slot_ok(s[0], false, "src") || !v.slot_ok(s[1], false, "dst") ||
          !v.holds(s[0], a[0], DT_F32, "src") || !v.holds(s[1], a[0], DT_F32, "dst") ||
          !v.writable(s[1], "dst"))
        return v.err;
      return SHK_HIP_STATUS_OK;
    case OP_TRANSPOSE:
      if (a[0] < 0 || a[1] < 0 || a[0] > INT32_MAX / 2 || a[1] > INT32_MAX / 2)
        return fail(SHK_HIP_STATUS_UNSUPPORTED_SHAPE, "step %zu: invalid transpose", idx);
      if (!v.slot_ok(s[0], false, "X") || !v.slot_ok(s[1], false, "Y") ||
          !v.holds(s[0], prod(a[0], a[1]), DT_F32, "X") || !v.holds(s[1], prod(a[0], a[1]), DT_F32, "Y") ||
          !v.writable(s[1], "Y"))
        return v.err;
      return SHK_HIP_STATUS_OK;
    default:
      return fail(SHK_HIP_STATUS_UNSUPPORTED_OPERATION, "step %zu: unknown opcode %u", idx, r.opcode);
  }
}

// ---- run-time dispatch ----
struct Bound {
  std::vector<void*> ptr;  // device pointer per slot
  template <typename T>
  T* get(int32_t s) const {
    return s < 0 || (size_t)s >= ptr.size() ? nullptr : static_cast<T*>(ptr[s]);
  }
};

// The optimizer launch parameters of an OP_OPTIMIZER step over the bound slots (null pointers
// for an empty binding: the tensor counts alone).
shk::OptParams optimizer_params(const Step& st, const Bound& b, uint32_t* status) {
  const StepRecord& r = st.rec;
  const int64_t* a = r.iarg;
  shk::OptParams p{};
  const OptEntry* e = reinterpret_cast<const OptEntry*>(st.payload.data());
  p.count = (int)(st.payload.size() / sizeof(OptEntry));
  for (int i = 0; i < p.count; ++i) {
    p.t[i].p = b.get<float>(e[i].p);
    p.t[i].g = b.get<const float>(e[i].g);
    p.t[i].m = b.get<float>(e[i].m);
    p.t[i].v = b.get<float>(e[i].v);
    p.t[i].pn = b.get<float>(e[i].pn);
    p.t[i].mn = b.get<float>(e[i].mn);
    p.t[i].vn = b.get<float>(e[i].vn);
    p.t[i].n = e[i].n;
  }
  p.kind = (int)a[0]; p.phase = (int)a[1]; p.nesterov = (int)a[2]; p.has_momentum_slot = (int)a[3];
  p.lr = r.farg[0]; p.momentum = r.farg[1]; p.dampening = r.farg[2]; p.weight_decay = r.farg[3];
  p.beta1 = r.farg[4]; p.beta2 = r.farg[5]; p.eps = r.farg[6];
  p.completed_steps = b.get<const int64_t>(r.slot[0]);
  p.status = status;
  return p;
}

hipError_t enqueue_step(const Step& st, const Bound& b, hipStream_t stream, double* scratch,
                        uint32_t* status) {
  const StepRecord& r = st.rec;
  const int32_t* s = r.slot;
  const int64_t* a = r.iarg;
  switch (r.opcode) {
    case OP_GEMM: {
      shk::GemmParams p{};
      p.A = b.get<const float>(s[0]);
      p.B = b.get<const float>(s[1]);
      p.C = b.get<float>(s[2]);
      p.bias = b.get<const float>(s[3]);
      p.aux = b.get<const float>(s[4]);
      p.M = a[0]; p.N = a[1]; p.K = a[2];
      p.lda = a[3]; p.ldb = a[4]; p.ldc = a[5]; p.ldaux = a[6];
      p.transA = (int)a[7]; p.transB = (int)a[8];
      p.act = (int)a[9]; p.mode = (int)a[10]; p.accumulate = (int)a[11];
      p.colsum = b.get<float>(s[5]);
      p.dz = b.get<float>(s[7]);
      if (!st.payload.empty()) {
        const OptEntry& e = *reinterpret_cast<const OptEntry*>(st.payload.data());
        shk::GemmUpdate& u = p.upd;
        u.p = b.get<const float>(e.p);
        u.m = b.get<const float>(e.m);
        u.v = b.get<const float>(e.v);
        u.pn = b.get<float>(e.pn);
        u.mn = b.get<float>(e.mn);
        u.vn = b.get<float>(e.vn);
        u.kind = (int)a[12]; u.nesterov = (int)a[13]; u.has_momentum_slot = (int)a[14];
        u.lr = r.farg[0]; u.momentum = r.farg[1]; u.dampening = r.farg[2]; u.weight_decay = r.farg[3];
        u.beta1 = r.farg[4]; u.beta2 = r.farg[5]; u.eps = r.farg[6];
        u.completed_steps = b.get<const int64_t>(s[6]);
        u.status = status;
      }
      return shk::launch_gemm(p, reinterpret_cast<float*>(scratch), stream);
    }
    case OP_COLSUM:
      return shk::launch_colsum(b.get<const float>(s[0]), b.get<float>(s[1]), a[0], a[1], a[2],
                                a[4] ? (double)a[0] : 1.0, (int)a[3], scratch, stream);
    case OP_ROW_REDUCE:
      return shk::launch_row_reduce(b.get<const float>(s[0]), b.get<float>(s[1]), a[0], a[1], (int)a[2], stream);
    case OP_REDUCE_ALL:
      return shk::launch_reduce_all(b.get<const float>(s[0]), b.get<float>(s[1]), a[0], (int)a[1],
                                    scratch, stream);
    case OP_POINTWISE: {
      shk::PwParams p{};
      for (int k = 0; k < shk::PW_MAX_INPUTS; ++k) {
        p.in[k] = b.get<const float>(s[k]);
        p.in_mode[k] = a[2 + k];
      }
      for (int o = 0; o < shk::PW_MAX_OUTPUTS; ++o) p.out[o] = b.get<float>(s[6 + o]);
      p.R = a[0]; p.C = a[1];
      p.n_instr = (int)(st.payload.size() / sizeof(shk::PwInstr));
      memcpy(p.code, st.payload.data(), st.payload.size());
      return shk::launch_pointwise(p, stream);
    }
    case OP_SOFTMAX:
      return shk::launch_softmax_fwd(b.get<const float>(s[0]), b.get<float>(s[1]), b.get<float>(s[2]),
                                     a[0], a[1], (int)a[2], stream);
    case OP_SOFTMAX_BWD:
      return shk::launch_softmax_bwd(b.get<const float>(s[0]), b.get<const float>(s[1]), b.get<float>(s[2]),
                                     a[0], a[1], b.get<const float>(s[3]), r.farg[0], stream);
    case OP_LSE_BWD:
      return shk::launch_lse_bwd(b.get<const float>(s[0]), b.get<const float>(s[1]), b.get<const float>(s[2]),
                                 r.farg[0], b.get<float>(s[3]), a[0], a[1], stream);
    case OP_MSE:
      return shk::launch_mse(b.get<const float>(s[0]), b.get<const float>(s[1]), b.get<float>(s[2]),
                             b.get<float>(s[3]), a[0], r.farg[0], (int)a[1], scratch, stream);
    case OP_CE_INDEX:
      return shk::launch_index_ce(b.get<const float>(s[0]), b.get<const void>(s[1]), (int)a[2],
                                  b.get<float>(s[2]), b.get<float>(s[3]), a[0], a[1], (int)a[3], a[4],
                                  r.farg[0], scratch, status, stream);
    case OP_CE_HEAD: {
      if (a[4] == 1) return shk::launch_ce_head_finish(b.get<const float>(s[0]), a[0], b.get<float>(s[1]), stream);
      shk::CeHeadParams p{};
      p.H = b.get<const float>(s[0]);
      p.W = b.get<const float>(s[1]);
      p.bias = b.get<const float>(s[2]);
      p.target = b.get<const void>(s[3]);
      p.logits = b.get<float>(s[4]);
      p.dz = b.get<float>(s[5]);
      p.dx = b.get<float>(s[6]);
      p.row_loss = b.get<float>(s[7]);
      p.status = status;
      p.R = a[0]; p.K = a[1]; p.J = (int)a[2]; p.act = (int)a[3]; p.target_is_64 = (int)a[5];
      p.g = r.farg[0];
      return shk::launch_ce_head(p, stream);
    }
    case OP_OPTIMIZER:
      return shk::launch_optimizer(optimizer_params(st, b, status), stream);
    case OP_STEP_COMMIT:
      return shk::launch_step_commit(b.get<int64_t>(s[0]), status, stream);
    case OP_FILL:
      return shk::launch_fill(b.get<float>(s[0]), a[0], r.farg[0], stream);
    case OP_COPY:
      return shk::launch_copy(b.get<const float>(s[0]), b.get<float>(s[1]), a[0], stream);
    case OP_TRANSPOSE:
      return shk::launch_transpose(b.get<const float>(s[0]), b.get<float>(s[1]), a[0], a[1], stream);
    default:
      return hipErrorInvalidValue;
  }
}

// Slots a step reads and writes, and whether it reads the status word (the step commit, the
// optimizer's apply phase and its accumulator commit / clear, which act only on a clear word) or
// only ORs bits into it (atomics: two such steps commute). Reduction scratch is not a slot: each
// stream has its own, and steps on one stream run in program order.
struct Access {
  std::vector<int32_t> r, w;
  bool status_read = false, status_or = false;
};
Access step_access(const Step& st) {
  const StepRecord& rec = st.rec;
  const int32_t* sl = rec.slot;
  const int64_t* a = rec.iarg;
  Access x;
  auto R = [&](int32_t v) { if (v >= 0) x.r.push_back(v); };
  auto W = [&](int32_t v) { if (v >= 0) x.w.push_back(v); };
  switch (rec.opcode) {
    case OP_GEMM:
      R(sl[0]); R(sl[1]); R(sl[3]); R(sl[4]); W(sl[2]); W(sl[5]); W(sl[7]);
      if (a[11]) R(sl[2]);  // accumulate
      if (!st.payload.empty()) {
        const OptEntry& e = *reinterpret_cast<const OptEntry*>(st.payload.data());
        R(e.p); R(e.m); R(e.v); W(e.pn); W(e.mn); W(e.vn); R(sl[6]);
        x.status_or = true;
      }
      break;
    case OP_COLSUM: R(sl[0]); W(sl[1]); if (a[3]) R(sl[1]); break;
    case OP_ROW_REDUCE: case OP_REDUCE_ALL: case OP_COPY: case OP_TRANSPOSE:
      R(sl[0]); W(sl[1]); break;
    case OP_POINTWISE:
      for (int k = 0; k < shk::PW_MAX_INPUTS; ++k) R(sl[k]);
      W(sl[6]); W(sl[7]);
      break;
    case OP_SOFTMAX: R(sl[0]); W(sl[1]); W(sl[2]); break;
    case OP_SOFTMAX_BWD: R(sl[0]); R(sl[1]); R(sl[3]); W(sl[2]); break;
    case OP_LSE_BWD: R(sl[0]); R(sl[1]); R(sl[2]); W(sl[3]); break;
    case OP_MSE: R(sl[0]); R(sl[1]); W(sl[2]); W(sl[3]); break;
    case OP_CE_INDEX: R(sl[0]); R(sl[1]); W(sl[2]); W(sl[3]); x.status_or = true; break;
    case OP_CE_HEAD:
      if (a[4] == 1) { R(sl[0]); W(sl[1]); break; }
      R(sl[0]); R(sl[1]); R(sl[2]); R(sl[3]); W(sl[4]); W(sl[5]); W(sl[6]); W(sl[7]);
      x.status_or = true;
      break;
    case OP_OPTIMIZER: {
      const OptEntry* e = reinterpret_cast<const OptEntry*>(st.payload.data());
      const size_t n = st.payload.size() / sizeof(OptEntry);
      for (size_t i = 0; i < n; ++i) {
        R(e[i].g); R(e[i].p); W(e[i].p); R(e[i].m); W(e[i].m); R(e[i].v); W(e[i].v);
        W(e[i].pn); W(e[i].mn); W(e[i].vn);
      }
      R(sl[0]);
      // the apply phase and the accumulator commit / clear act only when the status word is
      // clear: they read it, so they follow every step that can flag it
      if (a[1] == 1 || a[0] == 4 || a[0] == 5) x.status_read = true;
      if (a[0] == 3 || (a[0] <= 2 && a[1] != 1)) x.status_or = true;
      break;
    }
    case OP_STEP_COMMIT: R(sl[0]); W(sl[0]); x.status_read = true; break;
    case OP_FILL: W(sl[0]); break;
    default:  // unknown: conflicts with everything
      x.status_read = true;
      W(-2);
  }
  return x;
}
bool accesses_conflict(const Access& a, const Access& b) {
  auto meet = [](const std::vector<int32_t>& u, const std::vector<int32_t>& v) {
    for (int32_t p : u)
      for (int32_t q : v)
        if (p == q || p == -2 || q == -2) return true;
    return false;
  };
  return meet(a.w, b.r) || meet(a.w, b.w) || meet(a.r, b.w) ||
         (a.status_read && (b.status_or || b.status_read)) || (b.status_read && a.status_or);
}
bool concurrency_enabled() {
  static const bool on = [] {
    const char* e = std::getenv("SHK_HIP_CONCURRENT");
    return !(e != nullptr && e[0] == '0');
  }();
  return on;
}
// Two-stream list schedule: step j goes beside the main chain (stream 1) when it does not
// depend on the step currently at the tail of stream 0; a step waits (event) for every earlier
// step on the other stream it depends on. Steps on one stream keep program order.
// A GEMM with at least 2^28 multiply-adds: enough tiles to occupy every CU on its own.
bool large_gemm(const Step& st) {
  if (st.rec.opcode != OP_GEMM) return false;
  const int64_t* a = st.rec.iarg;
  if (a[0] <= 0 || a[1] <= 0 || a[2] <= 0) return false;
  const double macs = (double)a[0] * (double)a[1] * (double)a[2];
  return macs >= (double)(1ll << 28);
}

// Whether the two-stream plan is active by default: only for programs whose GEMMs total at
// least 2^28 multiply-adds. Each cross-stream event costs a few microseconds on the device
// (measured on MI355X: a 16 -> 64 -> 1 training step, 12 small kernels, takes 61 us on one stream
// and 80 us on two), which only steps long enough to hide side work beside them repay.
bool side_stream_pays(const Program& pr) {
  double macs = 0.0;
  for (const Step& st : pr.steps)
    if (st.rec.opcode == OP_GEMM) {
      const int64_t* a = st.rec.iarg;
      if (a[0] > 0 && a[1] > 0 && a[2] > 0) macs += (double)a[0] * (double)a[1] * (double)a[2];
    }
  return macs >= (double)(1ll << 28);
}

// Folding: the last OP_CE_HEAD finish step, and the last staged optimizer pass (phase 2, SGD /
// Adam / AdamW) of at most RUN_FINALE_MAX_OPT_BLOCKS blocks, whose accesses conflict with no
// later launched step's (nothing later reads what they write or writes what they read) move to
// the run's last launch, which performs them in program order after every launched step. Runs
// before plan_streams, which leaves folded steps out of the schedule. SHK_HIP_FOLD_FINISH=0 keeps
// every step a launch of its own.
void plan_fold(Program* pr) {
  static const bool on = [] {
    const char* e = std::getenv("SHK_HIP_FOLD_FINISH");
    return !(e != nullptr && e[0] == '0');
  }();
  pr->folded_finish = -1;
  pr->folded_opt = -1;
  const size_t n = pr->steps.size();
  const size_t launched = n > 0 && pr->steps[n - 1].rec.opcode == OP_STEP_COMMIT ? n - 1 : n;
  if (!on) return;
  auto last_foldable = [&](auto eligible) -> int64_t {
    for (size_t j = launched; j-- > 0;) {
      if (!eligible(pr->steps[j])) continue;
      const Access aj = step_access(pr->steps[j]);
      for (size_t k = j + 1; k < launched; ++k)
        if (!pr->folded(k) && accesses_conflict(aj, step_access(pr->steps[k]))) return -1;
      return (int64_t)j;
    }
    return -1;
  };
  static const int64_t max_elements = [] {
    const char* e = std::getenv("SHK_HIP_FOLD_OPT_MAX");
    return e != nullptr ? std::atoll(e) : (int64_t)1024;
  }();
  pr->folded_opt = last_foldable([](const Step& st) {
    const StepRecord& r = st.rec;
    if (r.opcode != OP_OPTIMIZER || r.iarg[1] != 2 || r.iarg[0] > 2) return false;
    const shk::OptParams p = optimizer_params(st, Bound(), nullptr);
    int64_t elements = 0;
    for (int i = 0; i < p.count; ++i) elements += p.t[i].n;
    return elements <= max_elements &&
           shk::optimizer_blocks(p) <= shk::RUN_FINALE_MAX_OPT_BLOCKS;
  });
  pr->folded_finish = last_foldable([](const Step& st) {
    return st.rec.opcode == OP_CE_HEAD && st.rec.iarg[4] == 1;
  });
}

void plan_streams(Program* pr) {
  const size_t n = pr->steps.size();
  pr->stream_of.assign(n, 0);
  pr->record_after.assign(n, 0);
  pr->wait_for.assign(n, {});
  pr->side_steps = 0;
  if (!concurrency_enabled() || n < 2) return;
  std::vector<Access> acc(n);
  for (size_t j = 0; j < n; ++j) acc[j] = step_access(pr->steps[j]);
  int64_t tail0 = -1;
  const size_t launched = pr->steps[n - 1].rec.opcode == OP_STEP_COMMIT ? n - 1 : n;
  // per stream: the latest step of the other stream its tail already follows (through a wait)
  int64_t covered[2] = {-1, -1};
  for (size_t j = 0; j < n; ++j) {
    // steps the publication kernel performs (folded ones, the trailing commit) follow the join
    // of both streams: they take no part in the schedule
    if (j >= launched || pr->folded(j)) continue;
    std::vector<uint32_t> deps;
    for (size_t i = 0; i < j; ++i)
      if (!pr->folded(i) && accesses_conflict(acc[i], acc[j])) deps.push_back((uint32_t)i);
    bool on_tail0 = tail0 < 0;
    for (uint32_t i : deps) on_tail0 |= (int64_t)i == tail0;
    // A large GEMM stays on the context stream even when it could run beside the chain: two
    // of them side by side take longer than one after the other (measured on MI355X: 1024^3 NN
    // and TN GEMMs, 46 us in sequence, 72 us on two streams), so the side stream carries only
    // the small steps that fill the gaps.
    const uint8_t sj = (on_tail0 || large_gemm(pr->steps[j])) ? 0 : 1;
    pr->stream_of[j] = sj;
    if (sj == 0) tail0 = (int64_t)j;
    // stream order covers same-stream dependencies and the other stream's earlier ones
    // behind its latest: one wait at most, none when an earlier wait on this stream covers it
    int64_t latest = -1;
    for (uint32_t i : deps)
      if (pr->stream_of[i] != sj) latest = std::max<int64_t>(latest, i);
    if (latest > covered[sj]) {
      covered[sj] = latest;
      pr->wait_for[j].push_back((uint32_t)latest);
      pr->record_after[latest] = 1;
    }
    if (sj == 1) pr->side_steps++;
  }
}

// Enqueues every step of one run on lease `ls`, then the status publication (copy to
// ls.host_status, clear): on stream s0 alone, or along the two-stream plan (fork from s0,
// per-dependency events, join back into s0). Profiling runs use s0 alone so that the per-step
// events bracket exactly one step each. A program whose last step is the step commit has it
// performed by the publication kernel: the commit reads the status word, so every step that can
// flag it precedes it, and nothing follows.
hipError_t enqueue_steps(const Program& pr, Lease& ls, const Bound& b, hipStream_t s0,
                         bool two_streams, bool profile, hipStream_t side = nullptr) {
  hipError_t e = hipSuccess;
  const size_t n = pr.steps.size();
  int64_t* commit = nullptr;
  if (n > 0 && pr.steps[n - 1].rec.opcode == OP_STEP_COMMIT)
    commit = b.get<int64_t>(pr.steps[n - 1].rec.slot[0]);
  const size_t launched = commit != nullptr ? n - 1 : n;
  // folded steps go into the run's last launch (not in profiled runs: their per-step events
  // bracket every step's own launch)
  auto skipped = [&](size_t j) { return !profile && pr.folded(j); };
  auto publish = [&]() -> hipError_t {
    shk::RunFinale f{};
    f.status = ls.status;
    f.host_word = ls.host_status;
    f.counter = commit;
    if (!profile && pr.folded_finish >= 0) {
      const StepRecord& r = pr.steps[(size_t)pr.folded_finish].rec;
      f.row_loss = b.get<const float>(r.slot[0]);
      f.R = r.iarg[0];
      f.loss = b.get<float>(r.slot[1]);
      f.mean_first = pr.folded_opt < 0 || pr.folded_finish < pr.folded_opt;
    }
    if (!profile && pr.folded_opt >= 0)
      f.opt = optimizer_params(pr.steps[(size_t)pr.folded_opt], b, ls.status);
    return shk::launch_run_finale(f, s0);
  };
  if (!two_streams || profile) {
    for (size_t i = 0; i < n; ++i) {
      if (profile && (e = hipEventRecord(ls.events[i], s0)) != hipSuccess) return e;
      if (i < launched && !skipped(i) &&
          (e = enqueue_step(pr.steps[i], b, s0, ls.scratch, ls.status)) != hipSuccess)
        return e;
    }
    if (profile && (e = hipEventRecord(ls.events[n], s0)) != hipSuccess) return e;
    return publish();
  }
  hipStream_t s1 = side != nullptr ? side : pr.ctx->side_stream;
  if ((e = hipEventRecord(ls.fork, s0)) != hipSuccess ||
      (e = hipStreamWaitEvent(s1, ls.fork, 0)) != hipSuccess)
    return e;
  for (size_t j = 0; j < launched; ++j) {
    if (skipped(j)) continue;  // no later step waits for it (plan_fold, plan_streams)
    const bool side = pr.stream_of[j] != 0;
    hipStream_t st = side ? s1 : s0;
    for (uint32_t i : pr.wait_for[j])
      if ((e = hipStreamWaitEvent(st, ls.step_done[i], 0)) != hipSuccess) return e;
    if ((e = enqueue_step(pr.steps[j], b, st, side ? ls.scratch_side : ls.scratch,
                          ls.status)) != hipSuccess)
      return e;
    if (pr.record_after[j] && (e = hipEventRecord(ls.step_done[j], st)) != hipSuccess) return e;
  }
  if ((e = hipEventRecord(ls.join, s1)) != hipSuccess) return e;
  if ((e = hipStreamWaitEvent(s0, ls.join, 0)) != hipSuccess) return e;
  return publish();
}

void destroy_lease(Lease* ls) {
  if (ls == nullptr) return;
  for (auto& kv : ls->graph_cache) (void)hipGraphExecDestroy(kv.second);
  for (hipEvent_t e : ls->events)
    if (e != nullptr) (void)hipEventDestroy(e);
  for (hipEvent_t e : ls->step_done)
    if (e != nullptr) (void)hipEventDestroy(e);
  if (ls->done != nullptr) (void)hipEventDestroy(ls->done);
  if (ls->cap0 != nullptr) (void)hipStreamDestroy(ls->cap0);
  if (ls->cap1 != nullptr) (void)hipStreamDestroy(ls->cap1);
  if (ls->fork != nullptr) (void)hipEventDestroy(ls->fork);
  if (ls->join != nullptr) (void)hipEventDestroy(ls->join);
  if (ls->host_status != nullptr) (void)hipHostFree(ls->host_status);
  if (ls->arena != nullptr) (void)hipFree(ls->arena);
  delete ls;
}

// Allocates one lease of `pr` (the device current): the zeroed arena, the pinned status word
// and the run's events. Returns the status and leaves *out null on failure.
int32_t create_lease(const Program& pr, Lease** out) {
  *out = nullptr;
  Lease* ls = new Lease();
  if (hipMalloc(&ls->arena, pr.arena_bytes) != hipSuccess) {
    ls->arena = nullptr;
    destroy_lease(ls);
    return fail(SHK_HIP_STATUS_ALLOCATION_FAILED, "program arena of %llu bytes failed",
                (unsigned long long)pr.arena_bytes);
  }
  // Internal slots start zeroed; a lease's later runs see what earlier runs on it left.
  if (hipMemset(ls->arena, 0, pr.arena_bytes) != hipSuccess) {
    destroy_lease(ls);
    return fail(SHK_HIP_STATUS_DEVICE_ERROR, "arena initialisation failed");
  }
  if (hipHostMalloc((void**)&ls->host_status, 16, hipHostMallocDefault) != hipSuccess) {
    ls->host_status = nullptr;
    destroy_lease(ls);
    return fail(SHK_HIP_STATUS_ALLOCATION_FAILED, "pinned status allocation failed");
  }
  bool ok = hipEventCreateWithFlags(&ls->done, hipEventDisableTiming) == hipSuccess;
  if (!ok) ls->done = nullptr;
  if (ok && hipStreamCreateWithFlags(&ls->cap0, hipStreamNonBlocking) != hipSuccess) {
    ls->cap0 = nullptr;
    ok = false;
  }
  if (ok && pr.side_steps > 0 &&
      hipStreamCreateWithFlags(&ls->cap1, hipStreamNonBlocking) != hipSuccess) {
    ls->cap1 = nullptr;
    ok = false;
  }
  ls->status = static_cast<uint32_t*>(ls->arena);
  ls->scratch = reinterpret_cast<double*>(static_cast<char*>(ls->arena) + pr.scratch_off);
  if (ok && pr.side_steps > 0) {
    ls->scratch_side = reinterpret_cast<double*>(static_cast<char*>(ls->arena) + pr.scratch_side_off);
    ok = hipEventCreateWithFlags(&ls->fork, hipEventDisableTiming) == hipSuccess;
    if (!ok) ls->fork = nullptr;
    ok = ok && hipEventCreateWithFlags(&ls->join, hipEventDisableTiming) == hipSuccess;
    if (!ok) ls->join = nullptr;
    ls->step_done.assign(pr.steps.size(), nullptr);
    for (size_t j = 0; ok && j < pr.steps.size(); ++j)
      if (pr.record_after[j] &&
          hipEventCreateWithFlags(&ls->step_done[j], hipEventDisableTiming) != hipSuccess) {
        ls->step_done[j] = nullptr;
        ok = false;
      }
  }
  if (!ok) {
    destroy_lease(ls);
    return fail(SHK_HIP_STATUS_DEVICE_ERROR, "event creation failed");
  }
  *out = ls;
  return SHK_HIP_STATUS_OK;
}

void destroy_program(Program* p) {
  if (p == nullptr) return;
  for (Lease* ls : p->leases) destroy_lease(ls);
  p->leases.clear();
  p->magic = 0;
  Context* c = p->ctx;
  delete p;
  if (c != nullptr) context_unref(c);
}

}  // namespace

extern "C" {

uint32_t shk_hip_abi_version(void) { return SHK_HIP_ABI_VERSION; }

int32_t shk_hip_last_error(char* destination, uint64_t capacity) {
  if (destination == nullptr || capacity == 0) return SHK_HIP_STATUS_INVALID_ARGUMENT;
  const size_t n = std::min<size_t>(capacity - 1, g_last_error.size());
  memcpy(destination, g_last_error.data(), n);
  destination[n] = '\0';
  return SHK_HIP_STATUS_OK;
}

int32_t shk_hip_context_create(int32_t device_ordinal, void** out_context) {
  if (out_context == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "out_context is null");
  *out_context = nullptr;
  try {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
      return fail(SHK_HIP_STATUS_NO_DEVICE, "no HIP device is available");
    if (device_ordinal < 0 || device_ordinal >= count)
      return fail(SHK_HIP_STATUS_NO_DEVICE, "device ordinal %d outside [0,%d)", device_ordinal, count);
    HIP_TRY(hipSetDevice(device_ordinal));
    resolve_static_scratch(device_ordinal);
    Context* c = new Context();
    c->device = device_ordinal;
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
      delete c;
      return fail(SHK_HIP_STATUS_NO_COMMAND_QUEUE, "hipStreamCreateWithFlags failed");
    }
    if (hipHostMalloc((void**)&c->host_status, 16, hipHostMallocDefault) != hipSuccess) {
      (void)hipStreamDestroy(c->stream);
      delete c;
      return fail(SHK_HIP_STATUS_ALLOCATION_FAILED, "pinned status allocation failed");
    }
    // The copy stream is created right after the compute stream, before any side stream, so
    // that the runtime gives it a hardware queue of its own (queues are handed out in stream
    // creation order): staged uploads must not queue behind compute work.
    if (hipStreamCreateWithFlags(&c->copy_stream, hipStreamNonBlocking) != hipSuccess) {
      (void)hipHostFree(c->host_status);
      (void)hipStreamDestroy(c->stream);
      delete c;
      return fail(SHK_HIP_STATUS_NO_COMMAND_QUEUE, "copy stream creation failed");
    }
    *out_context = c;
    return SHK_HIP_STATUS_OK;
  } catch (const std::bad_alloc&) {
    return fail(SHK_HIP_STATUS_ALLOCATION_FAILED, "host allocation failed");
  } catch (...) {
    return fail(SHK_HIP_STATUS_INTERNAL_ERROR, "unexpected exception");
  }
}

int32_t shk_hip_context_release(void* context) {
  Context* c = live_context(context);
  if (c == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "not a live context handle");
  if (c->released.exchange(true)) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "context already released");
  context_unref(c);
  return SHK_HIP_STATUS_OK;
}

int32_t shk_hip_device_info(void* context, int32_t* out_compute_units, int32_t* out_clock_khz,
                            uint64_t* out_memory_bytes, char* out_name, uint64_t name_capacity) {
  Context* c = live_context(context);
  if (c == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "not a context handle");
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, c->device));
  if (out_compute_units) *out_compute_units = prop.multiProcessorCount;
  if (out_clock_khz) *out_clock_khz = prop.clockRate;
  if (out_memory_bytes) *out_memory_bytes = prop.totalGlobalMem;
  if (out_name && name_capacity > 0) {
    const size_t n = std::min<size_t>(name_capacity - 1, strlen(prop.gcnArchName));
    memcpy(out_name, prop.gcnArchName, n);
    out_name[n] = '\0';
  }
  return SHK_HIP_STATUS_OK;
}

int32_t shk_hip_buffer_create(void* context, uint64_t byte_size, void** out_buffer) {
  if (out_buffer == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "out_buffer is null");
  *out_buffer = nullptr;
  Context* c = live_context(context);
  if (c == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "not a live context handle");
  try {
    HIP_TRY(hipSetDevice(c->device));
    void* p = nullptr;
    if (hipMalloc(&p, std::max<uint64_t>(byte_size, 256)) != hipSuccess)
      return fail(SHK_HIP_STATUS_ALLOCATION_FAILED, "hipMalloc of %llu bytes failed",
                  (unsigned long long)byte_size);
    Buffer* b = new Buffer();
    b->ctx = c;
    b->ptr = p;
    b->bytes = byte_size;
    c->refs.fetch_add(1);
    *out_buffer = b;
    return SHK_HIP_STATUS_OK;
  } catch (...) {
    return fail(SHK_HIP_STATUS_ALLOCATION_FAILED, "host allocation failed");
  }
}

int32_t shk_hip_buffer_wrap(void* context, void* device_pointer, uint64_t byte_size, void** out_buffer) {
  if (out_buffer == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "out_buffer is null");
  *out_buffer = nullptr;
  Context* c = live_context(context);
  if (c == nullptr || (device_pointer == nullptr && byte_size != 0))
    return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "invalid wrap arguments");
  try {
    Buffer* b = new Buffer();
    b->ctx = c;
    b->ptr = device_pointer;
    b->bytes = byte_size;
    b->owned = false;
    c->refs.fetch_add(1);
    *out_buffer = b;
    return SHK_HIP_STATUS_OK;
  } catch (...) {
    return fail(SHK_HIP_STATUS_ALLOCATION_FAILED, "host allocation failed");
  }
}

int32_t shk_hip_buffer_release(void* buffer) {
  Buffer* b = checked<Buffer, kBufferMagic>(buffer);
  if (b == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "not a buffer handle");
  (void)hipSetDevice(b->ctx->device);
  if (b->upload_pending) (void)hipEventSynchronize(b->upload_done);
  if (b->use_pending) (void)hipEventSynchronize(b->last_use);
  if (b->upload_done != nullptr) (void)hipEventDestroy(b->upload_done);
  if (b->last_use != nullptr) (void)hipEventDestroy(b->last_use);
  if (b->owned && b->ptr != nullptr) (void)hipFree(b->ptr);
  b->magic = 0;
  Context* c = b->ctx;
  delete b;
  context_unref(c);
  return SHK_HIP_STATUS_OK;
}

int32_t shk_hip_buffer_upload(void* buffer, uint64_t offset, const void* source, uint64_t byte_count) {
  Buffer* b = checked<Buffer, kBufferMagic>(buffer);
  if (b == nullptr || (source == nullptr && byte_count != 0))
    return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "invalid upload arguments");
  if (offset > b->bytes || byte_count > b->bytes - offset)
    return fail(SHK_HIP_STATUS_RANGE_OUT_OF_BOUNDS, "upload range outside the buffer");
  if (byte_count == 0) return SHK_HIP_STATUS_OK;
  std::lock_guard<std::mutex> lock(b->ctx->mutex);
  HIP_TRY(hipSetDevice(b->ctx->device));
  HIP_TRY(order_after_upload(b, b->ctx->stream));
  if (hipMemcpyAsync(static_cast<char*>(b->ptr) + offset, source, byte_count, hipMemcpyHostToDevice,
                     b->ctx->stream) != hipSuccess ||
      hipStreamSynchronize(b->ctx->stream) != hipSuccess)
    return fail(SHK_HIP_STATUS_COPY_FAILED, "host-to-device copy failed");
  return SHK_HIP_STATUS_OK;
}

int32_t shk_hip_buffer_download(void* buffer, uint64_t offset, void* destination, uint64_t byte_count) {
  Buffer* b = checked<Buffer, kBufferMagic>(buffer);
  if (b == nullptr || (destination == nullptr && byte_count != 0))
    return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "invalid download arguments");
  if (offset > b->bytes || byte_count > b->bytes - offset)
    return fail(SHK_HIP_STATUS_RANGE_OUT_OF_BOUNDS, "download range outside the buffer");
  if (byte_count == 0) return SHK_HIP_STATUS_OK;
  std::lock_guard<std::mutex> lock(b->ctx->mutex);
  HIP_TRY(hipSetDevice(b->ctx->device));
  HIP_TRY(order_after_upload(b, b->ctx->stream));
  if (hipMemcpyAsync(destination, static_cast<const char*>(b->ptr) + offset, byte_count,
                     hipMemcpyDeviceToHost, b->ctx->stream) != hipSuccess ||
      hipStreamSynchronize(b->ctx->stream) != hipSuccess)
    return fail(SHK_HIP_STATUS_COPY_FAILED, "device-to-host copy failed");
  return SHK_HIP_STATUS_OK;
}

}  // extern "C"

namespace {

// Grows the context's publication staging buffer (status word in its first 256 bytes, payload
// after it) to at least `need` bytes. Caller holds the context mutex with the device current.
int32_t ensure_pub_staging(Context* c, uint64_t need) {
  if (c->pub_staging_bytes >= need) return SHK_HIP_STATUS_OK;
  if (c->pub_staging != nullptr) {
    HIP_TRY(hipStreamSynchronize(c->stream));
    (void)hipFree(c->pub_staging);
    c->pub_staging = nullptr;
    c->pub_staging_bytes = 0;
  }
  if (hipMalloc((void**)&c->pub_staging, need) != hipSuccess) {
    c->pub_staging = nullptr;
    return fail(SHK_HIP_STATUS_ALLOCATION_FAILED, "publication staging of %llu bytes failed",
                (unsigned long long)need);
  }
  c->pub_staging_bytes = need;
  return SHK_HIP_STATUS_OK;
}

constexpr uint64_t kRingChunk = 8ull << 20;  // bytes per pinned staging chunk
constexpr int kRingSlots = 4;

// Creates the copy stream (default priority) and the pinned staging ring on first use (caller
// holds the context mutex with the device current).
int32_t ensure_copy_ring(Context* c) {
  if (c->copy_stream == nullptr &&
      hipStreamCreateWithFlags(&c->copy_stream, hipStreamNonBlocking) != hipSuccess) {
    c->copy_stream = nullptr;
    return fail(SHK_HIP_STATUS_NO_COMMAND_QUEUE, "copy stream creation failed");
  }
  for (int i = 0; i < kRingSlots; ++i) {  // (resumes where an earlier failed attempt stopped)
    if (c->ring[i] == nullptr &&
        hipHostMalloc((void**)&c->ring[i], kRingChunk, hipHostMallocDefault) != hipSuccess) {
      c->ring[i] = nullptr;
      return fail(SHK_HIP_STATUS_ALLOCATION_FAILED, "pinned staging chunk allocation failed");
    }
    if (c->ring_free[i] == nullptr &&
        hipEventCreateWithFlags(&c->ring_free[i], hipEventDisableTiming) != hipSuccess) {
      c->ring_free[i] = nullptr;
      return fail(SHK_HIP_STATUS_DEVICE_ERROR, "event creation failed");
    }
  }
  return SHK_HIP_STATUS_OK;
}

// Byte extent of a storage-layout transfer, or 0 when the geometry is not one
// (MetalBackendRuntime.isStorageTransfer / transferByteCount, MetalBackendRuntime.java:433-484;
// CpuMetalPreparedBufferTransfer.transferByteCount, CpuMetalPreparedBufferTransfer.java:79-127).
// The axes of extent > 1 are insertion-sorted by stride (a strictly larger stride moves ahead,
// so equal strides keep axis order); each must start at or beyond the element span the smaller
// ones cover, which rules out overlap. All arithmetic is checked signed 64-bit, as Java's
// Math.*Exact is.
uint64_t storage_transfer_extent(uint32_t width, uint32_t rank, const int64_t* dims,
                                 const int64_t* strides, int64_t offset) {
  if (width != 1 && width != 2 && width != 4 && width != 8) return 0;
  if (rank > (uint32_t)shk::CANONICAL_MAX_RANK || (rank > 0 && dims == nullptr) || offset < 0)
    return 0;
  int64_t st[shk::CANONICAL_MAX_RANK];
  if (strides == nullptr) {  // dense row-major
    int64_t e = 1;
    for (int a = (int)rank - 1; a >= 0; --a) {
      st[a] = e;
      if (dims[a] > 0 && __builtin_mul_overflow(e, dims[a], &e)) return 0;
    }
  } else {
    for (uint32_t a = 0; a < rank; ++a) st[a] = strides[a];
  }
  int64_t as[shk::CANONICAL_MAX_RANK], ad[shk::CANONICAL_MAX_RANK];
  int active = 0;
  for (uint32_t a = 0; a < rank; ++a) {
    if (dims[a] <= 0 || st[a] <= 0) return 0;
    if (dims[a] > 1) {
      int i = active;
      while (i > 0 && as[i - 1] > st[a]) {
        as[i] = as[i - 1];
        ad[i] = ad[i - 1];
        --i;
      }
      as[i] = st[a];
      ad[i] = dims[a];
      ++active;
    }
  }
  int64_t covered = 1;
  for (int i = 0; i < active; ++i) {
    if (as[i] < covered) return 0;
    int64_t ext;
    if (__builtin_mul_overflow(ad[i] - 1, as[i], &ext) ||
        __builtin_add_overflow(covered, ext, &covered))
      return 0;
  }
  int64_t span, bytes;
  if (__builtin_add_overflow(offset, covered, &span) ||
      __builtin_mul_overflow(span, (int64_t)width, &bytes) || bytes <= 0)
    return 0;
  return (uint64_t)bytes;
}

// Row-major ordinal walk over a view, calling f(storage element index) for each element.
template <typename F>
void for_each_storage_index(uint32_t rank, const int64_t* dims, const int64_t* strides,
                            int64_t offset, F f) {
  int64_t st[shk::CANONICAL_MAX_RANK], idx[shk::CANONICAL_MAX_RANK] = {};
  int64_t e = 1;
  for (int a = (int)rank - 1; a >= 0; --a) {
    st[a] = strides != nullptr ? strides[a] : e;
    e *= dims[a];
  }
  int64_t pos = offset;
  for (;;) {
    f(pos);
    int a = (int)rank - 1;
    for (; a >= 0; --a) {
      if (++idx[a] < dims[a]) {
        pos += st[a];
        break;
      }
      pos -= (dims[a] - 1) * st[a];
      idx[a] = 0;
    }
    if (a < 0) return;
  }
}

struct StorageTransfer {
  Buffer* b = nullptr;
  uint64_t bytes = 0;
};

// Shared argument checks of the two transfer directions (MetalBackendRuntime.java:211-265).
int32_t check_storage_transfer(void* buffer, uint32_t& width, int32_t boolean, uint32_t rank,
                               const int64_t* dims, const int64_t* strides, int64_t offset,
                               const void* host, uint64_t host_bytes, const char* side,
                               StorageTransfer* out) {
  Buffer* b = checked<Buffer, kBufferMagic>(buffer);
  if (b == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "not a buffer handle");
  if (b->ctx->released.load()) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "context is released");
  if (boolean) width = 1;
  const uint64_t bytes = storage_transfer_extent(width, rank, dims, strides, offset);
  if (bytes == 0)
    return fail(SHK_HIP_STATUS_INVALID_ARGUMENT,
                "storage transfer requires rank-0..16 static non-overlapping positive-stride "
                "geometry with a checked byte extent");
  if (b->bytes != bytes)
    return fail(SHK_HIP_STATUS_INVALID_ARGUMENT,
                "buffer byte size %llu does not match the transfer extent %llu",
                (unsigned long long)b->bytes, (unsigned long long)bytes);
  if (host == nullptr || host_bytes < bytes)
    return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "%s is smaller than its transfer extent", side);
  out->b = b;
  out->bytes = bytes;
  return SHK_HIP_STATUS_OK;
}

}  // namespace

extern "C" {

int32_t shk_hip_buffer_upload_staged(void* buffer, uint64_t offset, const void* source,
                                     uint64_t byte_count) {
  Buffer* b = checked<Buffer, kBufferMagic>(buffer);
  if (b == nullptr || (source == nullptr && byte_count != 0))
    return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "invalid upload arguments");
  if (b->ctx->released.load()) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "context is released");
  if (offset > b->bytes || byte_count > b->bytes - offset)
    return fail(SHK_HIP_STATUS_RANGE_OUT_OF_BOUNDS, "upload range outside the buffer");
  if (byte_count == 0) return SHK_HIP_STATUS_OK;
  Context* c = b->ctx;
  std::lock_guard<std::mutex> lock(c->mutex);
  HIP_TRY(hipSetDevice(c->device));
  {
    const int32_t st = ensure_copy_ring(c);
    if (st != SHK_HIP_STATUS_OK) return st;
  }
  if (b->upload_done == nullptr)
    HIP_TRY(hipEventCreateWithFlags(&b->upload_done, hipEventDisableTiming));
  // not before the last asynchronous run that bound this buffer has finished with it
  if (b->use_pending) HIP_TRY(hipStreamWaitEvent(c->copy_stream, b->last_use, 0));
  const uint8_t* src = static_cast<const uint8_t*>(source);
  uint8_t* dst = static_cast<uint8_t*>(b->ptr) + offset;
  for (uint64_t done = 0; done < byte_count;) {
    const uint64_t n = std::min<uint64_t>(kRingChunk, byte_count - done);
    const int slot = c->ring_next;
    c->ring_next = (c->ring_next + 1) % kRingSlots;
    if (c->ring_used[slot] && hipEventSynchronize(c->ring_free[slot]) != hipSuccess)
      return fail(SHK_HIP_STATUS_COPY_FAILED, "host-to-device copy failed");
    memcpy(c->ring[slot], src + done, n);
    if (hipMemcpyAsync(dst + done, c->ring[slot], n, hipMemcpyHostToDevice, c->copy_stream) !=
            hipSuccess ||
        hipEventRecord(c->ring_free[slot], c->copy_stream) != hipSuccess)
      return fail(SHK_HIP_STATUS_COPY_FAILED, "host-to-device copy failed");
    c->ring_used[slot] = true;
    done += n;
  }
  HIP_TRY(hipEventRecord(b->upload_done, c->copy_stream));
  b->upload_pending = true;
  return SHK_HIP_STATUS_OK;
}

int32_t shk_hip_storage_transfer_bytes(uint32_t element_width, uint32_t rank, const int64_t* dims,
                                       const int64_t* strides, int64_t storage_offset,
                                       uint64_t* out_bytes) {
  if (out_bytes == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "out_bytes is null");
  *out_bytes = storage_transfer_extent(element_width, rank, dims, strides, storage_offset);
  return SHK_HIP_STATUS_OK;
}

int32_t shk_hip_buffer_upload_storage(void* buffer, uint32_t element_width, int32_t boolean,
                                      uint32_t rank, const int64_t* dims, const int64_t* strides,
                                      int64_t storage_offset, const void* source,
                                      uint64_t source_bytes) {
  StorageTransfer t;
  int32_t st = check_storage_transfer(buffer, element_width, boolean, rank, dims, strides,
                                      storage_offset, source, source_bytes, "source", &t);
  if (st != SHK_HIP_STATUS_OK) return st;
  if (boolean) {  // MetalBackendRuntime.validateBooleanElements before the native write (:241-244)
    const uint8_t* p = static_cast<const uint8_t*>(source);
    bool bad = false;
    for_each_storage_index(rank, dims, strides, storage_offset,
                           [&](int64_t i) { bad |= p[i] > 1; });
    if (bad) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "BOOL source contains a non-canonical byte");
  }
  Context* c = t.b->ctx;
  std::lock_guard<std::mutex> lock(c->mutex);
  HIP_TRY(hipSetDevice(c->device));
  HIP_TRY(order_after_upload(t.b, c->stream));
  if (hipMemcpyAsync(t.b->ptr, source, t.bytes, hipMemcpyHostToDevice, c->stream) != hipSuccess ||
      hipStreamSynchronize(c->stream) != hipSuccess)
    return fail(SHK_HIP_STATUS_COPY_FAILED, "host-to-device copy failed");
  return SHK_HIP_STATUS_OK;
}

int32_t shk_hip_buffer_download_storage(void* buffer, uint32_t element_width, int32_t boolean,
                                        uint32_t rank, const int64_t* dims,
                                        const int64_t* strides, int64_t storage_offset,
                                        void* destination, uint64_t destination_capacity) {
  StorageTransfer t;
  int32_t st = check_storage_transfer(buffer, element_width, boolean, rank, dims, strides,
                                      storage_offset, destination, destination_capacity,
                                      "destination", &t);
  if (st != SHK_HIP_STATUS_OK) return st;
  Context* c = t.b->ctx;
  std::lock_guard<std::mutex> lock(c->mutex);
  HIP_TRY(hipSetDevice(c->device));
  HIP_TRY(order_after_upload(t.b, c->stream));
  if (boolean) {
    // Validation on the device before any byte reaches the destination (the reference downloads
    // into host staging and validates there, MetalBackendRuntime.java:270-281).
    st = ensure_pub_staging(c, 256);
    if (st != SHK_HIP_STATUS_OK) return st;
    shk::CanonicalGeometry g{};
    g.rank = (int32_t)rank;
    g.offset = storage_offset;
    int64_t elements = 1, e = 1;
    for (int a = (int)rank - 1; a >= 0; --a) {
      g.dims[a] = dims[a];
      g.strides[a] = strides != nullptr ? strides[a] : e;
      e *= dims[a];
      elements *= dims[a];
    }
    uint32_t* status = reinterpret_cast<uint32_t*>(c->pub_staging);
    HIP_TRY(shk::launch_fill_u32(status, 1, 0u, c->stream));
    HIP_TRY(shk::launch_bool_validate(t.b->ptr, elements, g, status, c->stream));
    HIP_TRY(hipMemcpyAsync(c->host_status, status, 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    if (*c->host_status & shk::DEV_INVALID_BOOL)
      return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "BOOL source contains a non-canonical byte");
  }
  if (hipMemcpyAsync(destination, t.b->ptr, t.bytes, hipMemcpyDeviceToHost, c->stream) !=
          hipSuccess ||
      hipStreamSynchronize(c->stream) != hipSuccess)
    return fail(SHK_HIP_STATUS_COPY_FAILED, "device-to-host copy failed");
  return SHK_HIP_STATUS_OK;
}

int32_t shk_hip_buffer_download_canonical(void* buffer, uint32_t element_width, int32_t boolean,
                                          uint32_t rank, const int64_t* dims,
                                          const int64_t* strides, int64_t storage_offset,
                                          void* destination, uint64_t destination_capacity,
                                          uint64_t maximum_bytes) {
  // Argument order and checks follow MetalBackendRuntime.copyToCanonicalHostBytes
  // (MetalBackendRuntime.java:304-357): payload limit, then the referenced storage span.
  Buffer* b = checked<Buffer, kBufferMagic>(buffer);
  if (b == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "not a buffer handle");
  if (b->ctx->released.load()) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "context is released");
  if (boolean) element_width = 1;
  if (element_width != 1 && element_width != 2 && element_width != 4 && element_width != 8)
    return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "element width must be 1, 2, 4 or 8");
  if (rank > (uint32_t)shk::CANONICAL_MAX_RANK || (rank > 0 && dims == nullptr))
    return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "rank must be 0..16 with dimensions");
  if (storage_offset < 0) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "negative storage offset");
  // element count and referenced span (LayoutGeometry.referencedElementSpan), overflow-checked
  uint64_t elements = 1, greatest = (uint64_t)storage_offset;
  bool empty = false;
  for (uint32_t a = 0; a < rank; ++a) {
    if (dims[a] < 0) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "negative dimension");
    if (strides != nullptr && strides[a] < 0)
      return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "negative stride");
    if (dims[a] == 0) empty = true;
  }
  for (uint32_t a = 0; a < rank && !empty; ++a) {
    if (__builtin_mul_overflow(elements, (uint64_t)dims[a], &elements))
      return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "element count overflows");
  }
  if (empty) elements = 0;
  uint64_t byte_count;
  if (__builtin_mul_overflow(elements, (uint64_t)element_width, &byte_count))
    return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "byte count overflows");
  if (byte_count > maximum_bytes)
    return fail(SHK_HIP_STATUS_INVALID_ARGUMENT,
                "canonical payload exceeds maximumBytes: required=%llu, maximum=%llu",
                (unsigned long long)byte_count, (unsigned long long)maximum_bytes);
  if (byte_count > destination_capacity || (destination == nullptr && byte_count != 0))
    return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "destination is smaller than the payload");
  uint64_t span = 0;  // referenced elements
  if (!empty) {
    if (strides == nullptr) {
      if (__builtin_add_overflow(greatest, elements, &span))
        return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "span overflows");
    } else {
      for (uint32_t a = 0; a < rank; ++a) {
        uint64_t ext;
        if (__builtin_mul_overflow((uint64_t)(dims[a] - 1), (uint64_t)strides[a], &ext) ||
            __builtin_add_overflow(greatest, ext, &greatest))
          return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "span overflows");
      }
      span = greatest + 1;
    }
  }
  uint64_t span_bytes;
  if (__builtin_mul_overflow(span, (uint64_t)element_width, &span_bytes) || span_bytes > b->bytes)
    return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "buffer is smaller than the descriptor's span");
  if (elements == 0) return SHK_HIP_STATUS_OK;

  // Dense from element 0: no gather. Otherwise the strided kernel with the view's geometry.
  bool dense = storage_offset == 0;
  if (strides != nullptr) {
    int64_t expect = 1;
    for (int a = (int)rank - 1; a >= 0 && dense; --a) {
      if (dims[a] != 1 && strides[a] != expect) dense = false;
      expect *= dims[a];
    }
  }
  shk::CanonicalGeometry g{};
  if (!dense) {
    g.rank = (int32_t)rank;
    g.offset = storage_offset;
    for (uint32_t a = 0; a < rank; ++a) {
      g.dims[a] = dims[a];
      g.strides[a] = strides != nullptr ? strides[a] : 0;
    }
    if (strides == nullptr) {  // dense row-major strides from a non-zero offset
      int64_t st = 1;
      for (int a = (int)rank - 1; a >= 0; --a) { g.strides[a] = st; st *= dims[a]; }
    }
  }
  Context* c = b->ctx;
  std::lock_guard<std::mutex> lock(c->mutex);
  HIP_TRY(hipSetDevice(c->device));
  HIP_TRY(order_after_upload(b, c->stream));
  // raw little-endian single bytes need no device pass
  if (dense && element_width == 1 && !boolean) {
    if (hipMemcpyAsync(destination, b->ptr, byte_count, hipMemcpyDeviceToHost, c->stream) !=
            hipSuccess ||
        hipStreamSynchronize(c->stream) != hipSuccess)
      return fail(SHK_HIP_STATUS_COPY_FAILED, "device-to-host copy failed");
    return SHK_HIP_STATUS_OK;
  }
  {
    const int32_t st = ensure_pub_staging(c, 256 + ((byte_count + 255) / 256) * 256);
    if (st != SHK_HIP_STATUS_OK) return st;
  }
  uint32_t* status = reinterpret_cast<uint32_t*>(c->pub_staging);
  uint8_t* packed = c->pub_staging + 256;
  HIP_TRY(shk::launch_fill_u32(status, 1, 0u, c->stream));
  HIP_TRY(shk::launch_canonical_pack(b->ptr, packed, (int64_t)elements, (int)element_width,
                                     boolean, dense ? nullptr : &g, status, c->stream));
  if (boolean) {
    HIP_TRY(hipMemcpyAsync(c->host_status, status, 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    if (*c->host_status & shk::DEV_INVALID_BOOL)
      return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "BOOL source contains a non-canonical byte");
  }
  if (hipMemcpyAsync(destination, packed, byte_count, hipMemcpyDeviceToHost, c->stream) !=
          hipSuccess ||
      hipStreamSynchronize(c->stream) != hipSuccess)
    return fail(SHK_HIP_STATUS_COPY_FAILED, "device-to-host copy failed");
  return SHK_HIP_STATUS_OK;
}

int32_t shk_hip_buffer_device_pointer(void* buffer, void** out_pointer) {
  if (out_pointer == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "out_pointer is null");
  *out_pointer = nullptr;
  Buffer* b = checked<Buffer, kBufferMagic>(buffer);
  if (b == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "not a buffer handle");
  *out_pointer = b->ptr;
  return SHK_HIP_STATUS_OK;
}

}  // extern "C"

namespace {

// Decodes and validates a program image into `pr` (slots, steps, the stream plan and the lease
// arena layout) without touching a device. Every step's operand extents are checked against its
// slots' byte sizes, dtypes and writability, so no launch of a created program can address
// outside a bound buffer.
int32_t decode_image(const void* image, uint64_t image_bytes, Program* pr) {
  const uint8_t* p = static_cast<const uint8_t*>(image);
  const uint8_t* end = p + image_bytes;
  if (image_bytes < sizeof(ImageHeader))
    return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "image shorter than its header");
  ImageHeader h;
  memcpy(&h, p, sizeof h);
  p += sizeof h;
  if (h.magic != kImageMagic || h.version != kImageVersion)
    return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "image magic/version mismatch");
  if (h.n_slots > 1u << 20 || h.n_steps > 1u << 20 ||
      (uint64_t)(end - p) < (uint64_t)h.n_slots * sizeof(SlotRecord))
    return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "image slot table truncated");
  pr->slots.resize(h.n_slots);
  memcpy(pr->slots.data(), p, h.n_slots * sizeof(SlotRecord));
  p += h.n_slots * sizeof(SlotRecord);
  std::vector<int> in_seen, out_seen;
  for (uint32_t i = 0; i < h.n_slots; ++i) {
    const SlotRecord& s = pr->slots[i];
    if (dtype_size(s.dtype) == 0 || s.kind > SLOT_INOUT)
      return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "slot %u has an invalid dtype or kind", i);
    if (s.kind != SLOT_INTERNAL && s.ext_index >= h.n_slots)
      return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "slot %u binding index out of range", i);
    if (s.kind == SLOT_INPUT || s.kind == SLOT_INOUT) {
      if (s.ext_index >= in_seen.size()) in_seen.resize(s.ext_index + 1, 0);
      in_seen[s.ext_index]++;
    } else if (s.kind == SLOT_OUTPUT) {
      if (s.ext_index >= out_seen.size()) out_seen.resize(s.ext_index + 1, 0);
      out_seen[s.ext_index]++;
    }
  }
  for (size_t i = 0; i < in_seen.size(); ++i)
    if (in_seen[i] != 1) {
      return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "input index %zu bound %d times", i, in_seen[i]);
    }
  for (size_t i = 0; i < out_seen.size(); ++i)
    if (out_seen[i] != 1) {
      return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "output index %zu bound %d times", i, out_seen[i]);
    }
  pr->n_inputs = (uint32_t)in_seen.size();
  pr->n_outputs = (uint32_t)out_seen.size();

  uint64_t scratch_doubles = 0;
  pr->steps.resize(h.n_steps);
  for (uint32_t i = 0; i < h.n_steps; ++i) {
    if ((uint64_t)(end - p) < sizeof(StepRecord)) {
      return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "image step %u truncated", i);
    }
    Step& st = pr->steps[i];
    memcpy(&st.rec, p, sizeof(StepRecord));
    p += sizeof(StepRecord);
    const uint64_t padded = (st.rec.payload_bytes + 7u) & ~7ull;
    if (st.rec.payload_bytes > 65536 || (uint64_t)(end - p) < padded) {
      return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "image step %u payload truncated", i);
    }
    st.payload.assign(p, p + st.rec.payload_bytes);
    p += padded;
    const int32_t v = validate_step(pr->slots, i, st, &scratch_doubles);
    if (v != SHK_HIP_STATUS_OK) return v;
  }
  if (p != end) return fail(SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED, "image has trailing bytes");

  // Lease arena layout: status word, reduction scratch (one per stream), then 256-byte
  // aligned internal slots.
  constexpr uint64_t kMaxArena = 1ull << 50;  // far beyond any device; keeps the sums exact
  if (scratch_doubles > kMaxArena / 8)
    return fail(SHK_HIP_STATUS_UNSUPPORTED_SHAPE, "reduction scratch too large");
  uint64_t off = 256;
  pr->scratch_off = off;
  off += ((scratch_doubles * 8 + 255) / 256) * 256;
  plan_fold(pr);
  plan_streams(pr);
  pr->scratch_side_off = off;
  if (pr->side_steps > 0) off += ((scratch_doubles * 8 + 255) / 256) * 256;
  pr->internal_offset.assign(h.n_slots, 0);
  for (uint32_t i = 0; i < h.n_slots; ++i) {
    if (pr->slots[i].kind != SLOT_INTERNAL) continue;
    if (pr->slots[i].bytes > kMaxArena || off > kMaxArena)
      return fail(SHK_HIP_STATUS_UNSUPPORTED_SHAPE, "internal slot %u too large", i);
    pr->internal_offset[i] = off;
    off += ((pr->slots[i].bytes + 255) / 256) * 256;
  }
  pr->arena_bytes = off;
  return SHK_HIP_STATUS_OK;
}

}  // namespace

extern "C" {

int32_t shk_hip_program_create(void* context, const void* image, uint64_t image_bytes, void** out_program) {
  if (out_program == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "out_program is null");
  *out_program = nullptr;
  Context* c = live_context(context);
  if (c == nullptr || image == nullptr)
    return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "invalid program arguments");
  Program* pr = nullptr;
  try {
    pr = new Program();
    pr->ctx = c;
    c->refs.fetch_add(1);
    const int32_t ds = decode_image(image, image_bytes, pr);
    if (ds != SHK_HIP_STATUS_OK) {
      destroy_program(pr);
      return ds;
    }
    pr->concurrent = pr->side_steps > 0 && side_stream_pays(*pr);
    if (pr->side_steps > 0) {
      std::lock_guard<std::mutex> lock(c->mutex);
      if (c->side_stream == nullptr &&
          (hipSetDevice(c->device) != hipSuccess ||
           hipStreamCreateWithFlags(&c->side_stream, hipStreamNonBlocking) != hipSuccess)) {
        c->side_stream = nullptr;
        destroy_program(pr);
        return fail(SHK_HIP_STATUS_NO_COMMAND_QUEUE, "side stream creation failed");
      }
    }
    {
      const char* e = getenv("SHK_HIP_MAX_LEASES");
      const long v = e != nullptr ? strtol(e, nullptr, 10) : 0;
      if (v >= 1 && v <= 64) pr->max_leases = (uint32_t)v;
    }
    // The first lease is allocated here, so that a program that runs one call at a time never
    // allocates device memory in a run.
    if (hipSetDevice(c->device) != hipSuccess) {
      destroy_program(pr);
      return fail(SHK_HIP_STATUS_DEVICE_ERROR, "hipSetDevice failed");
    }
    Lease* first = nullptr;
    const int32_t ls = create_lease(*pr, &first);
    if (ls != SHK_HIP_STATUS_OK) {
      destroy_program(pr);
      return ls;
    }
    pr->leases.push_back(first);
    pr->idle.push_back(first);
    pr->step_ms.assign(pr->steps.size(), 0.0);
    {
      const char* g = getenv("SHK_HIP_GRAPHS");
      // A program of large GEMMs only launches step by step by default: each launch is hidden
      // behind the previous kernel, and graph replay adds a few microseconds per node (C2's
      // fused layer: 0.404 ms direct, 0.410 ms replayed). So does a program of at most five
      // launched steps: a synchronous run replayed as a graph costs about 30 us whatever its
      // length up to 16 kernels, launched directly about 14 us plus 2.5 us per kernel (measured
      // on MI355X with chains of 1 to 16 copy steps: 16 / 22 / 27 / 38 / 53 us direct against
      // 32 / 37 / 33 / 36 / 45 us replayed for 1 / 2 / 4 / 8 / 16 steps).
      bool all_large = !pr->steps.empty();
      size_t launched = 0;
      for (size_t j = 0; j < pr->steps.size(); ++j) {
        all_large = all_large && large_gemm(pr->steps[j]);
        launched += !pr->folded(j) && pr->steps[j].rec.opcode != OP_STEP_COMMIT;
      }
      pr->graphs = !(g != nullptr && g[0] == '0') && !all_large && launched > 5;
    }
    *out_program = pr;
    return SHK_HIP_STATUS_OK;
  } catch (const std::bad_alloc&) {
    destroy_program(pr);
    return fail(SHK_HIP_STATUS_ALLOCATION_FAILED, "host allocation failed");
  } catch (...) {
    destroy_program(pr);
    return fail(SHK_HIP_STATUS_INTERNAL_ERROR, "unexpected exception");
  }
}

int32_t shk_hip_program_validate(const void* image, uint64_t image_bytes,
                                 uint64_t* out_arena_bytes) {
  if (out_arena_bytes != nullptr) *out_arena_bytes = 0;
  if (image == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "image is null");
  try {
    Program pr;  // decoded and discarded; no context, no device
    const int32_t st = decode_image(image, image_bytes, &pr);
    if (st == SHK_HIP_STATUS_OK && out_arena_bytes != nullptr) *out_arena_bytes = pr.arena_bytes;
    pr.magic = 0;
    return st;
  } catch (const std::bad_alloc&) {
    return fail(SHK_HIP_STATUS_ALLOCATION_FAILED, "host allocation failed");
  } catch (...) {
    return fail(SHK_HIP_STATUS_INTERNAL_ERROR, "unexpected exception");
  }
}

int32_t shk_hip_program_plan(const void* image, uint64_t image_bytes, uint32_t capacity,
                             uint8_t* out_stream, int32_t* out_wait, int64_t* out_folded,
                             uint32_t* out_steps) {
  if (out_steps != nullptr) *out_steps = 0;
  if (out_folded != nullptr) out_folded[0] = out_folded[1] = -1;
  if (image == nullptr || out_steps == nullptr)
    return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "image or out_steps is null");
  try {
    Program pr;  // decoded and discarded; no context, no device
    const int32_t st = decode_image(image, image_bytes, &pr);
    pr.magic = 0;
    if (st != SHK_HIP_STATUS_OK) return st;
    const size_t n = pr.steps.size();
    *out_steps = (uint32_t)n;
    if (out_folded != nullptr) {
      out_folded[0] = pr.folded_finish;
      out_folded[1] = pr.folded_opt;
    }
    if (capacity < n || out_stream == nullptr || out_wait == nullptr)
      return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "plan of %zu steps needs that capacity", n);
    for (size_t j = 0; j < n; ++j) {
      out_stream[j] = pr.stream_of[j];
      if (pr.wait_for[j].size() > 1)
        return fail(SHK_HIP_STATUS_INTERNAL_ERROR, "step %zu waits for more than one event", j);
      out_wait[j] = pr.wait_for[j].empty() ? -1 : (int32_t)pr.wait_for[j][0];
    }
    return SHK_HIP_STATUS_OK;
  } catch (const std::bad_alloc&) {
    return fail(SHK_HIP_STATUS_ALLOCATION_FAILED, "host allocation failed");
  } catch (...) {
    return fail(SHK_HIP_STATUS_INTERNAL_ERROR, "unexpected exception");
  }
}

int32_t shk_hip_program_release(void* program) {
  Program* pr = checked<Program, kProgramMagic>(program);
  if (pr == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "not a program handle");
  {
    std::lock_guard<std::mutex> lock(pr->ctx->mutex);
    (void)hipSetDevice(pr->ctx->device);
    (void)hipStreamSynchronize(pr->ctx->stream);
    if (pr->ctx->side_stream != nullptr) (void)hipStreamSynchronize(pr->ctx->side_stream);
  }
  destroy_program(pr);
  return SHK_HIP_STATUS_OK;
}

int32_t shk_hip_program_arena_bytes(void* program, uint64_t* out_bytes) {
  Program* pr = checked<Program, kProgramMagic>(program);
  if (pr == nullptr || out_bytes == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "invalid arguments");
  *out_bytes = pr->arena_bytes;
  return SHK_HIP_STATUS_OK;
}

int32_t shk_hip_program_lease_count(void* program, uint32_t* out_leases) {
  Program* pr = checked<Program, kProgramMagic>(program);
  if (pr == nullptr || out_leases == nullptr)
    return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "invalid arguments");
  std::lock_guard<std::mutex> lock(pr->mutex);
  *out_leases = (uint32_t)pr->leases.size();
  return SHK_HIP_STATUS_OK;
}

}  // extern "C"

namespace {

// Observes the completion of the run held on `ls` and maps its status word, then returns the
// lease to the pool. The caller holds no lock. Accumulates the run's step times when it was
// profiled.
int32_t finish_lease(Program* pr, Lease* ls, bool profiled) {
  const hipError_t se = hipEventSynchronize(ls->done);
  int32_t status = SHK_HIP_STATUS_OK;
  if (se != hipSuccess) {
    ls->status_clear = false;
    status = fail(SHK_HIP_STATUS_EXECUTION_FAILED, "program execution failed: %s",
                  hipGetErrorName(se));
  } else {
    const uint32_t st = *ls->host_status;
    if (st & shk::DEV_INDEX_OUT_OF_BOUNDS)
      status = fail(SHK_HIP_STATUS_INDEX_OUT_OF_BOUNDS, "index target out of bounds");
    else if (st & shk::DEV_NOT_POSITIVE)
      status = fail(SHK_HIP_STATUS_ARITHMETIC,
                    "adaptive bias correction or denominator is not positive");
    else if (st & shk::DEV_NON_FINITE)
      status = fail(SHK_HIP_STATUS_ARITHMETIC, "optimizer intermediate or candidate is not finite");
  }
  std::vector<float> ms;
  if (profiled && se == hipSuccess) {
    ms.resize(pr->steps.size(), 0.f);
    for (size_t i = 0; i < pr->steps.size(); ++i)
      if (hipEventElapsedTime(&ms[i], ls->events[i], ls->events[i + 1]) != hipSuccess) ms[i] = 0.f;
  }
  std::lock_guard<std::mutex> lock(pr->mutex);
  if (!ms.empty()) {
    for (size_t i = 0; i < ms.size(); ++i) pr->step_ms[i] += ms[i];
    pr->profiled_runs++;
  }
  pr->idle.push_back(ls);
  pr->lease_freed.notify_one();
  return status;
}

// Completes every asynchronous run of the program not yet waited for, oldest first, and returns
// the first failure among them. The caller holds pr->mutex (released while waiting).
int32_t finish_pending_locked(Program* pr, std::unique_lock<std::mutex>& lock) {
  int32_t first = SHK_HIP_STATUS_OK;
  std::string first_msg;
  while (!pr->pending.empty()) {
    Lease* ls = pr->pending.front();
    pr->pending.erase(pr->pending.begin());
    const bool profiled = !ls->events.empty() && pr->profiling;
    lock.unlock();
    const int32_t st = finish_lease(pr, ls, profiled);
    if (st != SHK_HIP_STATUS_OK && first == SHK_HIP_STATUS_OK) {
      first = st;
      first_msg = g_last_error;
    }
    lock.lock();
  }
  if (first != SHK_HIP_STATUS_OK) g_last_error = first_msg;
  return first;
}

// Takes an idle lease, or creates one while fewer than max_leases exist, or waits for one to be
// returned. The caller holds pr->mutex through `lock`.
int32_t acquire_lease(Program* pr, std::unique_lock<std::mutex>& lock, Lease** out) {
  *out = nullptr;
  for (;;) {
    if (!pr->idle.empty()) {
      *out = pr->idle.back();
      pr->idle.pop_back();
      return SHK_HIP_STATUS_OK;
    }
    if (pr->leases.size() < pr->max_leases) {
      // Under the context mutex: allocation and the synchronous arena clear must not run while
      // another thread captures a run's HIP graph on the context stream (captures hold it).
      std::lock_guard<std::mutex> ctx_lock(pr->ctx->mutex);
      HIP_TRY(hipSetDevice(pr->ctx->device));
      Lease* ls = nullptr;
      const int32_t st = create_lease(*pr, &ls);
      if (st != SHK_HIP_STATUS_OK) return st;
      pr->leases.push_back(ls);
      *out = ls;
      return SHK_HIP_STATUS_OK;
    }
    pr->lease_freed.wait(lock);
  }
}

void return_lease(Program* pr, Lease* ls) {
  std::lock_guard<std::mutex> lock(pr->mutex);
  pr->idle.push_back(ls);
  pr->lease_freed.notify_one();
}

// Binds, validates and enqueues one run on a lease of its own; synchronous runs then wait for
// it, asynchronous ones return with it pending. Asynchronous runs of the program not yet waited
// for are completed first, and the first failure among them is returned without launching.
// Checks the caller's bindings of a run and fills the external slots of `b` (internal slots
// stay null); `bound` receives every bound buffer. Sizes, contexts and aliasing are validated.
int32_t bind_external(Program* pr, uint32_t input_count, void* const* inputs,
                      uint32_t output_count, void* const* outputs, Bound* b,
                      std::vector<Buffer*>* bound) {
  if (input_count != pr->n_inputs || output_count != pr->n_outputs)
    return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "program expects %u inputs and %u outputs, got %u and %u",
                pr->n_inputs, pr->n_outputs, input_count, output_count);
  if ((input_count && inputs == nullptr) || (output_count && outputs == nullptr))
    return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "null binding array");
  std::vector<Buffer*> in(input_count), out(output_count);
  for (uint32_t i = 0; i < input_count; ++i) {
    in[i] = checked<Buffer, kBufferMagic>(inputs[i]);
    if (in[i] == nullptr || in[i]->ctx != pr->ctx)
      return fail(SHK_HIP_STATUS_INCOMPATIBLE_RESOURCE, "input %u is not a buffer of this context", i);
  }
  for (uint32_t i = 0; i < output_count; ++i) {
    out[i] = checked<Buffer, kBufferMagic>(outputs[i]);
    if (out[i] == nullptr || out[i]->ctx != pr->ctx)
      return fail(SHK_HIP_STATUS_INCOMPATIBLE_RESOURCE, "output %u is not a buffer of this context", i);
  }
  b->ptr.assign(pr->slots.size(), nullptr);
  std::vector<std::pair<uintptr_t, uintptr_t>> written;  // [begin,end) of outputs and in-place inputs
  std::vector<std::pair<uintptr_t, uintptr_t>> all;
  for (size_t i = 0; i < pr->slots.size(); ++i) {
    const SlotRecord& s = pr->slots[i];
    if (s.kind == SLOT_INTERNAL) continue;  // bound to the run's arena by the caller
    Buffer* buf = s.kind == SLOT_OUTPUT ? out[s.ext_index] : in[s.ext_index];
    if (buf->bytes < s.bytes)
      return fail(SHK_HIP_STATUS_INCOMPATIBLE_RESOURCE, "slot %zu needs %llu bytes, bound buffer has %llu", i,
                  (unsigned long long)s.bytes, (unsigned long long)buf->bytes);
    b->ptr[i] = buf->ptr;
    const uintptr_t lo = reinterpret_cast<uintptr_t>(buf->ptr), hi = lo + std::max<uint64_t>(s.bytes, 1);
    if (s.kind != SLOT_INPUT) written.push_back({lo, hi});
    all.push_back({lo, hi});
  }
  // A written buffer may not overlap any other bound buffer (Metal: synaptik_metal_foundation.m:10012-10020).
  for (const auto& w : written) {
    int overlaps = 0;
    for (const auto& o : all)
      if (o.first < w.second && w.first < o.second) ++overlaps;
    if (overlaps > 1)
      return fail(SHK_HIP_STATUS_INCOMPATIBLE_RESOURCE, "an output or in-place input aliases another binding");
  }
  bound->assign(in.begin(), in.end());
  bound->insert(bound->end(), out.begin(), out.end());
  return SHK_HIP_STATUS_OK;
}

// Binds, validates and enqueues one run on a lease of its own; synchronous runs then wait for
// it, asynchronous ones return with it pending. Asynchronous runs of the program not yet waited
// for are completed first, and the first failure among them is returned without launching.
int32_t run_program(void* program, uint32_t input_count, void* const* inputs, uint32_t output_count,
                    void* const* outputs, bool async) {
  Program* pr = checked<Program, kProgramMagic>(program);
  if (pr == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "not a program handle");
  try {
    Bound b;
    std::vector<Buffer*> bound;
    const int32_t bs = bind_external(pr, input_count, inputs, output_count, outputs, &b, &bound);
    if (bs != SHK_HIP_STATUS_OK) return bs;

    Lease* ls = nullptr;
    bool graphs, two_streams, profile;
    {
      std::unique_lock<std::mutex> lock(pr->mutex);
      const int32_t st = finish_pending_locked(pr, lock);
      if (st != SHK_HIP_STATUS_OK) return st;
      const int32_t la = acquire_lease(pr, lock, &ls);
      if (la != SHK_HIP_STATUS_OK) return la;
      graphs = pr->graphs && ls->graphs_ok;
      two_streams = pr->concurrent;
      profile = pr->profiling;
    }
    for (size_t i = 0; i < pr->slots.size(); ++i)
      if (pr->slots[i].kind == SLOT_INTERNAL)
        b.ptr[i] = static_cast<char*>(ls->arena) + pr->internal_offset[i];

    std::unique_lock<std::mutex> ctx_lock(pr->ctx->mutex);
    auto give_back = [&](int32_t status) {
      ctx_lock.unlock();
      return_lease(pr, ls);
      return status;
    };
    if (hipSetDevice(pr->ctx->device) != hipSuccess)
      return give_back(fail(SHK_HIP_STATUS_DEVICE_ERROR, "hipSetDevice failed"));
    if (profile && ls->events.empty()) {
      ls->events.assign(pr->steps.size() + 1, nullptr);
      for (auto& e : ls->events)
        if (hipEventCreate(&e) != hipSuccess) {
          e = nullptr;
          for (auto& x : ls->events)
            if (x != nullptr) (void)hipEventDestroy(x);
          ls->events.clear();
          return give_back(fail(SHK_HIP_STATUS_DEVICE_ERROR, "event creation failed"));
        }
    }
    hipStream_t stream = pr->ctx->stream;
    for (Buffer* x : bound)  // staged uploads landed
      if (order_after_upload(x, stream) != hipSuccess)
        return give_back(fail(SHK_HIP_STATUS_DEVICE_ERROR, "waiting for a staged upload failed"));
    if (!ls->status_clear) {
      // not cleared by a completed run's publication; from here until this run completes, a
      // failure leaves it unknown again
      if (shk::launch_fill_u32(ls->status, 4, 0u, stream) != hipSuccess)
        return give_back(fail(SHK_HIP_STATUS_EXECUTION_FAILED, "status clear failed"));
    }
    ls->status_clear = false;
    bool launched = false;
    if (graphs && !profile) {
      // cache key: the bound pointers, then the schedule (one stream / two streams)
      std::vector<void*> key(b.ptr);
      key.push_back(reinterpret_cast<void*>(static_cast<uintptr_t>(two_streams ? 2 : 1)));
      auto it = ls->graph_cache.find(key);
      if (it == ls->graph_cache.end()) {
        // capture: every step + the status publication (kernels only, no memset or copy node)
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        // captured on the lease's private streams, launched on the context stream below
        bool ok = hipStreamBeginCapture(ls->cap0, hipStreamCaptureModeRelaxed) == hipSuccess;
        if (ok) {
          const bool steps_ok =
              enqueue_steps(*pr, *ls, b, ls->cap0, two_streams, false, ls->cap1) == hipSuccess;
          const bool ended = hipStreamEndCapture(ls->cap0, &graph) == hipSuccess;
          ok = steps_ok && ended && graph != nullptr &&
               hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) == hipSuccess;
          if (graph != nullptr) (void)hipGraphDestroy(graph);
        }
        (void)hipGetLastError();  // a failed capture falls back to direct launches
        if (ok) {
          if (ls->graph_order.size() >= 8) {
            auto old = ls->graph_cache.find(ls->graph_order.front());
            if (old != ls->graph_cache.end()) {
              (void)hipGraphExecDestroy(old->second);
              ls->graph_cache.erase(old);
            }
            ls->graph_order.erase(ls->graph_order.begin());
          }
          it = ls->graph_cache.emplace(key, exec).first;
          ls->graph_order.push_back(key);
        } else {
          if (exec != nullptr) (void)hipGraphExecDestroy(exec);
          ls->graphs_ok = false;
        }
      }
      if (it != ls->graph_cache.end()) {
        if (hipGraphLaunch(it->second, stream) != hipSuccess)
          return give_back(fail(SHK_HIP_STATUS_EXECUTION_FAILED, "graph launch failed"));
        launched = true;
      }
    }
    if (!launched) {
      const hipError_t e = enqueue_steps(*pr, *ls, b, stream, two_streams, profile);
      if (e != hipSuccess) {
        (void)hipStreamSynchronize(stream);
        if (pr->ctx->side_stream != nullptr) (void)hipStreamSynchronize(pr->ctx->side_stream);
        return give_back(fail(SHK_HIP_STATUS_EXECUTION_FAILED, "step launch failed: %s",
                              hipGetErrorName(e)));
      }
    }
    if (hipEventRecord(ls->done, stream) != hipSuccess) {
      (void)hipStreamSynchronize(stream);
      return give_back(fail(SHK_HIP_STATUS_DEVICE_ERROR, "event record failed"));
    }
    ls->status_clear = true;  // once `done` completes without error
    if (async) {
      // a later staged upload into any bound buffer waits for this run (write-after-read)
      for (Buffer* x : bound) {
        if (x->last_use == nullptr &&
            hipEventCreateWithFlags(&x->last_use, hipEventDisableTiming) != hipSuccess) {
          x->last_use = nullptr;
          (void)hipStreamSynchronize(stream);
          return give_back(fail(SHK_HIP_STATUS_DEVICE_ERROR, "event creation failed"));
        }
        if (hipEventRecord(x->last_use, stream) != hipSuccess) {
          (void)hipStreamSynchronize(stream);
          return give_back(fail(SHK_HIP_STATUS_DEVICE_ERROR, "event record failed"));
        }
        x->use_pending = true;
      }
      ctx_lock.unlock();
      std::lock_guard<std::mutex> lock(pr->mutex);
      pr->pending.push_back(ls);
      return SHK_HIP_STATUS_OK;
    }
    ctx_lock.unlock();
    return finish_lease(pr, ls, profile);
  } catch (const std::bad_alloc&) {
    return fail(SHK_HIP_STATUS_ALLOCATION_FAILED, "host allocation failed");
  } catch (...) {
    return fail(SHK_HIP_STATUS_INTERNAL_ERROR, "unexpected exception");
  }
}

// The no-allocation run: the arena of the run (status word, reduction scratch, internal slots)
// is this device's copy of `scratch`, cleared by a fill kernel first; the steps run on the
// context stream alone, launched directly (no graph is captured or instantiated, no event is
// created), and the run's status is published to the context's pinned word. The device's static
// run mutex and then the context mutex are held from the arena clear until the stream has
// drained, so two runs that share one device's array never overlap, whichever contexts they go
// through.
int32_t run_static(void* program, uint32_t input_count, void* const* inputs,
                   uint32_t output_count, void* const* outputs) {
  Program* pr = checked<Program, kProgramMagic>(program);
  if (pr == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "not a program handle");
  if (pr->arena_bytes > kStaticScratchBytes)
    return fail(SHK_HIP_STATUS_UNSUPPORTED_SHAPE,
                "the program needs %llu bytes of per-run device memory (status word, reduction "
                "scratch and internal slots); shk_hip_program_run_static holds at most %llu",
                (unsigned long long)pr->arena_bytes, (unsigned long long)kStaticScratchBytes);
  const int device = pr->ctx->device;
  void* base = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (device >= 0 && device < kMaxDevices) base = g_scratch_address[device];
    if (base == nullptr)
      return fail(SHK_HIP_STATUS_DEVICE_ERROR, "static scratch of device %d unavailable: %s", device,
                  hipGetErrorName(device >= 0 && device < kMaxDevices ? g_scratch_error[device]
                                                                      : hipErrorInvalidDevice));
  }
  try {
    Bound b;
    std::vector<Buffer*> bound;
    const int32_t bs = bind_external(pr, input_count, inputs, output_count, outputs, &b, &bound);
    if (bs != SHK_HIP_STATUS_OK) return bs;
    {
      std::unique_lock<std::mutex> lock(pr->mutex);
      const int32_t st = finish_pending_locked(pr, lock);
      if (st != SHK_HIP_STATUS_OK) return st;
    }
    char* arena = static_cast<char*>(base);
    for (size_t i = 0; i < pr->slots.size(); ++i)
      if (pr->slots[i].kind == SLOT_INTERNAL) b.ptr[i] = arena + pr->internal_offset[i];
    Lease view;  // the lease-shaped view of the static arena (owns nothing)
    view.arena = arena;
    view.status = reinterpret_cast<uint32_t*>(arena);
    view.scratch = reinterpret_cast<double*>(arena + pr->scratch_off);
    view.host_status = pr->ctx->host_status;

    // device lock first, then the context's: no path takes them in the other order
    std::lock_guard<std::mutex> device_lock(g_static_run_mutex[device]);
    std::lock_guard<std::mutex> ctx_lock(pr->ctx->mutex);
    HIP_TRY(hipSetDevice(device));
    hipStream_t stream = pr->ctx->stream;
    for (Buffer* x : bound) HIP_TRY(order_after_upload(x, stream));  // staged uploads landed
    // The array keeps the last run's contents: clear the status word, the scratch and the
    // internal slots, so this run sees what a fresh lease would.
    hipError_t e = shk::launch_fill_u32(view.status, (int64_t)(pr->arena_bytes / 4), 0u, stream);
    if (e == hipSuccess) e = enqueue_steps(*pr, view, b, stream, false, false);
    const hipError_t se = hipStreamSynchronize(stream);
    if (e != hipSuccess)
      return fail(SHK_HIP_STATUS_EXECUTION_FAILED, "step launch failed: %s", hipGetErrorName(e));
    if (se != hipSuccess)
      return fail(SHK_HIP_STATUS_EXECUTION_FAILED, "program execution failed: %s", hipGetErrorName(se));
    const uint32_t st = *view.host_status;
    if (st & shk::DEV_INDEX_OUT_OF_BOUNDS)
      return fail(SHK_HIP_STATUS_INDEX_OUT_OF_BOUNDS, "index target out of bounds");
    if (st & shk::DEV_NOT_POSITIVE)
      return fail(SHK_HIP_STATUS_ARITHMETIC, "adaptive bias correction or denominator is not positive");
    if (st & shk::DEV_NON_FINITE)
      return fail(SHK_HIP_STATUS_ARITHMETIC, "optimizer intermediate or candidate is not finite");
    return SHK_HIP_STATUS_OK;
  } catch (const std::bad_alloc&) {
    return fail(SHK_HIP_STATUS_ALLOCATION_FAILED, "host allocation failed");
  } catch (...) {
    return fail(SHK_HIP_STATUS_INTERNAL_ERROR, "unexpected exception");
  }
}

// Applies a settings change with every pending asynchronous run completed first.
template <typename F>
int32_t with_settings(void* program, F f) {
  Program* pr = checked<Program, kProgramMagic>(program);
  if (pr == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "not a program handle");
  std::unique_lock<std::mutex> lock(pr->mutex);
  const int32_t st = finish_pending_locked(pr, lock);
  if (st != SHK_HIP_STATUS_OK) return st;
  return f(pr);
}
}  // namespace

extern "C" {

int32_t shk_hip_program_set_graph_mode(void* program, int32_t enabled) {
  return with_settings(program, [&](Program* pr) {
    pr->graphs = enabled != 0;
    return (int32_t)SHK_HIP_STATUS_OK;
  });
}

int32_t shk_hip_program_graph_mode(void* program, int32_t* out_enabled) {
  if (out_enabled == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "out_enabled is null");
  *out_enabled = 0;
  return with_settings(program, [&](Program* pr) {
    *out_enabled = pr->graphs ? 1 : 0;
    return (int32_t)SHK_HIP_STATUS_OK;
  });
}

int32_t shk_hip_program_set_concurrent(void* program, int32_t enabled) {
  // captured graphs embed the schedule; the graph cache key includes it, so both stay cached
  return with_settings(program, [&](Program* pr) {
    pr->concurrent = enabled != 0 && pr->side_steps > 0;
    return (int32_t)SHK_HIP_STATUS_OK;
  });
}

int32_t shk_hip_program_side_steps(void* program, uint32_t* out_steps) {
  Program* pr = checked<Program, kProgramMagic>(program);
  if (pr == nullptr || out_steps == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "invalid arguments");
  std::lock_guard<std::mutex> lock(pr->mutex);
  *out_steps = pr->concurrent ? pr->side_steps : 0;
  return SHK_HIP_STATUS_OK;
}

int32_t shk_hip_program_step_count(void* program, uint32_t* out_steps) {
  Program* pr = checked<Program, kProgramMagic>(program);
  if (pr == nullptr || out_steps == nullptr) return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "invalid arguments");
  *out_steps = (uint32_t)pr->steps.size();
  return SHK_HIP_STATUS_OK;
}

int32_t shk_hip_program_set_profiling(void* program, int32_t enabled) {
  return with_settings(program, [&](Program* pr) {
    pr->profiling = enabled != 0;
    pr->profiled_runs = 0;
    std::fill(pr->step_ms.begin(), pr->step_ms.end(), 0.0);
    return (int32_t)SHK_HIP_STATUS_OK;
  });
}

int32_t shk_hip_program_step_times(void* program, double* out_milliseconds, uint32_t capacity,
                                   uint64_t* out_runs) {
  if (out_milliseconds == nullptr && capacity != 0)
    return fail(SHK_HIP_STATUS_INVALID_ARGUMENT, "invalid arguments");
  return with_settings(program, [&](Program* pr) {
    for (uint32_t i = 0; i < capacity && i < pr->step_ms.size(); ++i)
      out_milliseconds[i] = pr->step_ms[i];
    if (out_runs) *out_runs = pr->profiled_runs;
    return (int32_t)SHK_HIP_STATUS_OK;
  });
}

int32_t shk_hip_program_run(void* program, uint32_t input_count, void* const* inputs,
                            uint32_t output_count, void* const* outputs) {
  return run_program(program, input_count, inputs, output_count, outputs, false);
}

int32_t shk_hip_program_run_async(void* program, uint32_t input_count, void* const* inputs,
                                  uint32_t output_count, void* const* outputs) {
  return run_program(program, input_count, inputs, output_count, outputs, true);
}

int32_t shk_hip_program_run_static(void* program, uint32_t input_count, void* const* inputs,
                                   uint32_t output_count, void* const* outputs) {
  return run_static(program, input_count, inputs, output_count, outputs);
}

int32_t shk_hip_program_wait(void* program) {
  return with_settings(program, [](Program*) { return (int32_t)SHK_HIP_STATUS_OK; });
}

}  // extern "C"
