/*
 * synaptik_hip.h - C ABI of the Synaptik MI355X (gfx950) execution backend, libsynaptik_hip.so.
 *
 * This is the native seam a Java `HipNativeApi` binds over the JDK 26 Foreign Function & Memory
 * API, exactly as the Metal backend binds libsynaptik_metal
 * (modules/backend/metal/src/main/java/io/github/pho001/synaptik/backend/metal/MetalNativeApi.java:3582-3700;
 *  exports in modules/backend/metal/macos-arm64/src/synaptik_metal_foundation.m:1681-1770,8573,9984-10160).
 *
 * Conventions (same as the Metal ABI):
 *   - every entry point returns an int32 status (SHK_HIP_STATUS_*), never throws, and NULLs its
 *     out-pointer on entry;
 *   - handles are opaque, owned by the caller's wrapper and released exactly once;
 *   - calls may come from any thread; a context serializes the work it enqueues on its stream;
 *     concurrent runs of one program are isolated: each holds a per-run lease of its own (see
 *     shk_hip_program_create);
 *   - a program run is synchronous: device work is complete when it returns
 *     (docs/architecture/contracts/backend-execution.md:1658-1660).
 * The last error message of the calling thread is available through shk_hip_last_error().
 */
#ifndef SYNAPTIK_HIP_H
#define SYNAPTIK_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SHK_HIP_ABI_VERSION 1u

/* Status vocabulary: 0-13 are the Metal ABI's codes with the same meaning
 * (synaptik_metal_foundation.m:74-87, mapped to Java exceptions in MetalNativeApi.java:482-507).
 * 14-16 are HIP additions. */
enum {
    SHK_HIP_STATUS_OK = 0,
    SHK_HIP_STATUS_INVALID_ARGUMENT = 1,
    SHK_HIP_STATUS_NO_DEVICE = 2,
    SHK_HIP_STATUS_NO_COMMAND_QUEUE = 3,
    SHK_HIP_STATUS_ALLOCATION_FAILED = 4,
    SHK_HIP_STATUS_RANGE_OUT_OF_BOUNDS = 5,
    SHK_HIP_STATUS_COPY_FAILED = 6,
    SHK_HIP_STATUS_INTERNAL_ERROR = 7,
    SHK_HIP_STATUS_UNSUPPORTED_SHAPE = 8,
    SHK_HIP_STATUS_GRAPH_COMPILATION_FAILED = 9,
    SHK_HIP_STATUS_INCOMPATIBLE_RESOURCE = 10,
    SHK_HIP_STATUS_EXECUTION_FAILED = 11,
    SHK_HIP_STATUS_KERNEL_COMPILATION_FAILED = 12,
    SHK_HIP_STATUS_UNSUPPORTED_OPERATION = 13,
    /* a HIP runtime call failed; the message carries the hipError_t name */
    SHK_HIP_STATUS_DEVICE_ERROR = 14,
    /* an optimizer intermediate was not finite or an adaptive denominator / bias correction
     * was not positive: nothing was committed (Java: ArithmeticException,
     * TrainingParameter.java:488-525) */
    SHK_HIP_STATUS_ARITHMETIC = 15,
    /* a categorical target index lay outside the class extent (Java: IllegalArgumentException,
     * CpuLossReferenceKernel.java:264) */
    SHK_HIP_STATUS_INDEX_OUT_OF_BOUNDS = 16
};

/* ABI version; a binding refuses a library with another value
 * (Metal: synaptik_metal_abi_version, MetalNativeApi.java:3655). */
uint32_t shk_hip_abi_version(void);

/* Copies the calling thread's last error message (NUL-terminated, truncated to capacity). */
int32_t shk_hip_last_error(char* destination, uint64_t capacity);

/* Context = one device + one stream. Replaces synaptik_metal_context_create/_release
 * (synaptik_metal_foundation.m:1683-1708). */
int32_t shk_hip_context_create(int32_t device_ordinal, void** out_context);
int32_t shk_hip_context_release(void* context);
/* Device facts for roofline reporting: compute units, peak engine clock (kHz), HBM bytes. */
int32_t shk_hip_device_info(void* context, int32_t* out_compute_units, int32_t* out_clock_khz,
                            uint64_t* out_memory_bytes, char* out_name, uint64_t name_capacity);

/* Device buffers. Replace synaptik_metal_buffer_create/_release/_upload/_download
 * (synaptik_metal_foundation.m:1710-1770). Uploads and downloads are synchronous. */
int32_t shk_hip_buffer_create(void* context, uint64_t byte_size, void** out_buffer);
/* Wraps caller-owned device memory (not freed on release). */
int32_t shk_hip_buffer_wrap(void* context, void* device_pointer, uint64_t byte_size,
                            void** out_buffer);
int32_t shk_hip_buffer_release(void* buffer);
int32_t shk_hip_buffer_upload(void* buffer, uint64_t offset, const void* source, uint64_t byte_count);
int32_t shk_hip_buffer_download(void* buffer, uint64_t offset, void* destination, uint64_t byte_count);
int32_t shk_hip_buffer_device_pointer(void* buffer, void** out_pointer);
/* Staged upload of caller host memory (pageable or not): the bytes are copied through a ring of
 * context-owned pinned chunks and moved by DMA on a second stream of the context, so the copy
 * overlaps device work. Returns once the source has been read in full (it may be reused) and the
 * last DMA is enqueued. Ordering: every later use of the buffer through this library (a run, a
 * download, an upload, a transfer) waits for the DMA; the DMA waits for the last asynchronous
 * run that bound the buffer. Replaces the pageable upload behind the reference's per-run borrow
 * of host tensors (MetalBackendRuntime.borrow, MetalBackendRuntime.java:173-200) when batches
 * stream in from the host; a HIP addition for pinned staging. */
int32_t shk_hip_buffer_upload_staged(void* buffer, uint64_t offset, const void* source,
                                     uint64_t byte_count);
/* Canonical host publication. Replaces the host-side packing of
 * MetalBackendRuntime.copyToCanonicalHostBytes (modules/backend/metal/src/main/java/io/github/
 * pho001/synaptik/backend/metal/MetalBackendRuntime.java:304-424, HostTensorValue.java:18):
 * writes the rank-`rank` view of `buffer` (dims; element strides, NULL = dense row-major;
 * storage_offset in elements) to destination as dense row-major bytes, every multi-byte element
 * big-endian with its raw bits kept. element_width is 1, 2, 4 or 8; boolean != 0 marks BOOL
 * (one byte per element), whose elements must be 0 or 1 (otherwise INVALID_ARGUMENT and nothing
 * is written). Checks, in the reference's order: payload bytes > maximum_bytes
 * (INVALID_ARGUMENT), payload > destination_capacity, referenced span beyond the buffer,
 * rank > 16, negative extents / strides / offset (all INVALID_ARGUMENT). An empty view returns
 * OK without device work. The packing is one device pass into a context-owned staging buffer
 * followed by one device-to-host copy; the call is synchronous. */
int32_t shk_hip_buffer_download_canonical(void* buffer, uint32_t element_width, int32_t boolean,
                                          uint32_t rank, const int64_t* dims,
                                          const int64_t* strides, int64_t storage_offset,
                                          void* destination, uint64_t destination_capacity,
                                          uint64_t maximum_bytes);

/* Storage-layout transfers: the physical referenced span of a typed view, moved byte for byte
 * between host memory and a device buffer of exactly that size (prefix and gap bytes included,
 * uninterpreted). Replace the Metal sides of the prepared CPU/device buffer transfer
 * (MetalBackendRuntime.acceptsStorageLayoutTransfer / bindStorageLayoutUpload /
 * bindStorageLayoutDownload, MetalBackendRuntime.java:211-281, used by
 * CpuMetalPreparedBufferTransfer.java:185-249). The geometry must be a storage transfer
 * (MetalBackendRuntime.isStorageTransfer, :433-478): rank 0..16, every extent and stride
 * positive (strides NULL = dense row-major), the axes with extent > 1 sorted by stride each
 * starting at or beyond the span the smaller ones cover (no overlap), span = storage_offset +
 * covered elements, and span * element_width representable as a positive int64.
 *
 * shk_hip_storage_transfer_bytes writes that byte extent to *out_bytes, or 0 when the geometry
 * is not a storage transfer; it touches no device. */
int32_t shk_hip_storage_transfer_bytes(uint32_t element_width, uint32_t rank, const int64_t* dims,
                                       const int64_t* strides, int64_t storage_offset,
                                       uint64_t* out_bytes);
/* Host -> device. INVALID_ARGUMENT when the geometry is not a storage transfer, the buffer's
 * byte size differs from the extent, or source_bytes is smaller than it; boolean != 0 (BOOL,
 * element_width 1): every logical element of the source must be 0 or 1, checked on the host
 * before anything is copied. Synchronous. */
int32_t shk_hip_buffer_upload_storage(void* buffer, uint32_t element_width, int32_t boolean,
                                      uint32_t rank, const int64_t* dims, const int64_t* strides,
                                      int64_t storage_offset, const void* source,
                                      uint64_t source_bytes);
/* Device -> host, same checks with destination_capacity. For BOOL every logical element is
 * validated on the device first; on a non-canonical byte the call fails with INVALID_ARGUMENT
 * and the destination is not written. Synchronous. */
int32_t shk_hip_buffer_download_storage(void* buffer, uint32_t element_width, int32_t boolean,
                                        uint32_t rank, const int64_t* dims,
                                        const int64_t* strides, int64_t storage_offset,
                                        void* destination, uint64_t destination_capacity);

/* Programs: an op-list image (the HIP analogue of the Metal graph image decoded by
 * synaptik_metal_mpsgraph_executable_create, synaptik_metal_foundation.m:8573). The decoded
 * program is immutable and shared by every run, as the reference's PreparedExecutable is
 * (PreparedExecutable.java:58-186). Per-run state -- a device arena with the internal slots,
 * the reduction scratch and the status word, plus the run's events and captured HIP graphs --
 * lives in leases owned by the program, the analogue of RunState-owned buffers and workspaces
 * (docs/backend-guide/writing-a-backend.md:140-142): a run holds one lease until its
 * completion is observed, and concurrent runs hold different leases, so their results are those
 * of running them one after another (Engine.java:480-507). The first lease is allocated here;
 * a run that finds every lease held creates another, up to 4 per program (SHK_HIP_MAX_LEASES,
 * 1..64, read here), and beyond that waits for one to be returned. A lease's internal slots
 * start zeroed and keep what its last run left. Image layout: synaptik_amd/program.py and
 * runtime.cpp. */
int32_t shk_hip_program_create(void* context, const void* image, uint64_t image_bytes,
                               void** out_program);
int32_t shk_hip_program_release(void* program);
/* Decodes and validates an image exactly as shk_hip_program_create does, without a context or a
 * device, and writes the per-run arena bytes one lease of the program would take
 * (shk_hip_program_arena_bytes) -- the Workspace requirement a preparer reports at analysis
 * time. HIP addition; returns the status shk_hip_program_create would for a malformed image. */
int32_t shk_hip_program_validate(const void* image, uint64_t image_bytes,
                                 uint64_t* out_arena_bytes);
/* Runs the program once: binds in[i] / out[i] to the image's input / output slots by index,
 * validates sizes and aliasing (INCOMPATIBLE_RESOURCE), enqueues every step, waits, and maps
 * the device status word (ARITHMETIC, INDEX_OUT_OF_BOUNDS). Replaces
 * synaptik_metal_mpsgraph_executable_run (synaptik_metal_foundation.m:9984-10083).
 * Runs from several threads proceed concurrently on different leases; their kernels are
 * enqueued on the context's streams one run after another. */
int32_t shk_hip_program_run(void* program, uint32_t input_count, void* const* inputs,
                            uint32_t output_count, void* const* outputs);
/* shk_hip_program_run without the wait: binds, validates and enqueues the run, then returns;
 * shk_hip_program_wait completes every pending asynchronous run of the program, oldest first,
 * and maps their status words exactly as shk_hip_program_run would (the first failure is
 * returned). A run, set_profiling, set_graph_mode, set_concurrent or step_times call on a
 * program with pending asynchronous runs first completes them, and returns the first failure
 * among them without doing anything else.
 * HIP addition (the reference's BoundInvocation.executeBound is synchronous): it lets a host
 * batch upload (shk_hip_buffer_upload_staged) overlap the previous run. */
int32_t shk_hip_program_run_async(void* program, uint32_t input_count, void* const* inputs,
                                  uint32_t output_count, void* const* outputs);
int32_t shk_hip_program_wait(void* program);
/* shk_hip_program_run without device allocation. No counterpart in the reference: a HIP
 * addition for callers that cannot allocate device memory (code under HIP-graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). The run's per-run device memory (status word,
 * reduction scratch, internal slots: shk_hip_program_arena_bytes) lives in a file-scope device
 * array of the library, one 64 MiB copy per device, held until the process ends; a program
 * needing more is refused with UNSUPPORTED_SHAPE. The call acquires no lease, captures no HIP
 * graph and creates no event or buffer: it clears the array with a kernel, launches the steps
 * on the context stream (the one-stream order), waits, and maps the status word as
 * shk_hip_program_run does. Pending asynchronous runs of the program are completed first.
 * Calls that use one device's array are serialized by a per-device lock, whichever contexts
 * they go through (a call waits for the one in progress); the array keeps the last call's
 * contents and each call clears it first. Results equal shk_hip_program_run's on a fresh lease. */
int32_t shk_hip_program_run_static(void* program, uint32_t input_count, void* const* inputs,
                                   uint32_t output_count, void* const* outputs);
/* The two-stream step schedule shk_hip_program_create would give an image, without a context or a
 * device (HIP addition, for schedule checks): per step its stream (0 = the context stream, 1 = the
 * side stream) and the one earlier step of the other stream it waits for (-1: none), and in
 * out_folded[0..1] the steps the run's last launch performs instead of launches of their own: the
 * loss MEAN of a fused classifier head and a small staged optimizer pass (-1: none). Steps keep
 * program order on each stream; every side step starts after the run's fork from the context
 * stream, and the last launch (folded steps in program order, the trailing step commit, the
 * status publication) follows the join of both; folded steps and the trailing commit have no
 * stream entry of their own (stream 0, no wait). out_steps receives the step count even when
 * `capacity` is too small (INVALID_ARGUMENT). SHK_HIP_CONCURRENT=0 gives the one-stream plan. */
int32_t shk_hip_program_plan(const void* image, uint64_t image_bytes, uint32_t capacity,
                             uint8_t* out_stream, int32_t* out_wait, int64_t* out_folded,
                             uint32_t* out_steps);
/* Two-stream step schedule (HIP addition; planned at creation unless SHK_HIP_CONCURRENT=0): each
 * step's slot reads and writes give its dependencies, and a step that does not depend on the step
 * at the tail of the context stream runs beside it on a second stream of the context (its own
 * reduction scratch), joined back by events -- e.g. the input- and weight-gradient GEMMs of one
 * layer. Results are those of the one-stream order. The plan is active by default only for
 * programs whose GEMMs total at least 2^28 multiply-adds: each cross-stream event costs a few
 * microseconds on the device, more than overlap gains for smaller programs. set_concurrent(0)
 * runs every step on the context stream, (1) activates the plan; side_steps reports how many
 * steps the active plan puts on the second stream. */
int32_t shk_hip_program_set_concurrent(void* program, int32_t enabled);
int32_t shk_hip_program_side_steps(void* program, uint32_t* out_steps);
/* Arena bytes of one lease (internal slots + scratch + status word). */
int32_t shk_hip_program_arena_bytes(void* program, uint64_t* out_bytes);
/* Number of leases the program has created (1 after create; more after concurrent runs).
 * HIP addition for observability. */
int32_t shk_hip_program_lease_count(void* program, uint32_t* out_leases);
/* Per-step device timing with HIP events on the context stream. Enabling clears the totals. */
int32_t shk_hip_program_set_profiling(void* program, int32_t enabled);
/* Writes min(capacity, steps) accumulated milliseconds per step and the number of profiled runs. */
int32_t shk_hip_program_step_times(void* program, double* out_milliseconds, uint32_t capacity,
                                   uint64_t* out_runs);
int32_t shk_hip_program_step_count(void* program, uint32_t* out_steps);
/* HIP-graph replay of the whole step sequence: each distinct set of bound buffers is captured
 * once and replayed with one launch. The default is on, except for a program whose every step
 * is a GEMM large enough to occupy the device (at least 2^28 multiply-adds): there the launches
 * are hidden behind the previous kernel anyway and replay only adds per-node cost; and for a
 * program of at most five launched steps, whose direct launches cost less than a replay's
 * fixed cost. SHK_HIP_GRAPHS=0 turns the default off. Profiled runs always launch step by step. */
int32_t shk_hip_program_set_graph_mode(void* program, int32_t enabled);
/* The current graph-replay setting (HIP addition). */
int32_t shk_hip_program_graph_mode(void* program, int32_t* out_enabled);

#ifdef __cplusplus
}
#endif

#endif /* SYNAPTIK_HIP_H */
