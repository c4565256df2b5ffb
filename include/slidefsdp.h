/*
 * slidefsdp.h -- C ABI of the MI355X layer-streaming library.
 *
 * Two shared libraries implement this header:
 *   libsf_hip.so  device kernels, copies and pinned host memory (HIP, gfx950)
 *   libsf_cpu.so  the host AdamW used by LayerAdam (C++, AVX-512 + OpenMP)
 *                 and the storage offload engine (C++, worker threads)
 *
 * Conventions shared by every entry point:
 *   - Plain pointers and sizes only; no framework types cross this boundary.
 *   - Return 0 on success. Nonzero values are either a hipError_t or one of
 *     the SF_E* codes below; sf_error_string() turns any of them into text.
 *   - Device entry points are asynchronous on the caller's stream, allocate
 *     nothing and keep no global mutable state, so any host thread may call
 *     them concurrently on different streams.  The one exception is
 *     sf_stage_f32_bf16_noalloc, whose device scratch buffer is shared by
 *     all its calls on a device: the library orders each call after the
 *     previous one on that device (an event it records), whatever stream
 *     each runs on.
 *   - Sizes are element counts unless the name says bytes.
 *
 * Each declaration names the reference interface (file:line in the
 * SlideFSDP sources) whose work it takes over.
 */
#ifndef SLIDEFSDP_H
#define SLIDEFSDP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* An opaque HIP stream handle (hipStream_t); 0 is the null stream. */
typedef void* sf_stream_t;
/* A HIP event (hipEvent_t), created by sf_event_create. */
typedef void* sf_event_t;

/* Library-specific status codes, disjoint from hipError_t values. */
#define SF_OK 0
#define SF_EINVAL 9001      /* null pointer, negative count, bad enum */
#define SF_ETOOMANY 9002    /* more segments than SF_MAX_SEGS in one call */
#define SF_EDTYPE 9003      /* dtype combination not supported */
#define SF_ENOOPT 9004      /* unknown optimizer id */
#define SF_EOVERLAP 9005    /* source and destination ranges overlap */
#define SF_ENOREQ 9006      /* unknown or already released I/O ticket */
#define SF_EALIGN 9007      /* O_DIRECT transfer not aligned to SF_IO_ALIGN */
#define SF_ETOOBIG 9008     /* larger than the library's device scratch */
#define SF_ETIMEDOUT 9009   /* a bounded wait ended before the work completed */
#define SF_EDMA_BASE 10000  /* + (hsa_status_t & 0xFFF): a ROCr DMA call failed */
#define SF_EIO_BASE 20000   /* + errno: a file operation failed */

/* Maximum number of segments one segment-table call accepts. */
#define SF_MAX_SEGS 64

/* One contiguous run of n elements copied from src to dst.  Both are
 * absolute addresses (device or host-mapped); n counts elements of the
 * entry point's element type. */
typedef struct sf_seg {
    uint64_t src;
    uint64_t dst;
    uint64_t n;
} sf_seg;

/* ---------------------------------------------------------------------
 * Status and version
 * ------------------------------------------------------------------- */

/* Text for any status returned by this library (never NULL). */
const char* sf_error_string(int status);

/* ABI version, bumped on any incompatible change (SF_ABI_VERSION).
 * 2: row_slot markers of the row-wise AdamW (SF_ROW_SKIP; other values
 *    below SF_ROW_SKIP are an error).
 * 3: sf_dma_wait takes a deadline (timeout_ns; SF_ETIMEDOUT). */
#define SF_ABI_VERSION 3
int sf_abi_version(void);

/* ---------------------------------------------------------------------
 * Parameter staging (libsf_hip.so)
 * ------------------------------------------------------------------- */

/* fp32 -> bf16, round to nearest even, NaN -> 0xFFFF, dst[i] = rne(src[i])
 * for i < n.  Replaces the host-side cast of the flat fp32 master into the
 * pinned bf16 convert buffer, layer_state.py:301
 * (`_bf16_convert_buffer[:total_size].copy_(_cpu_params_flat)`); here it
 * runs in HBM after the fp32 master has been copied to the device. */
int sf_cast_f32_bf16(const float* src, uint16_t* dst, size_t n,
                     sf_stream_t stream);

/* sf_cast_f32_bf16 with `start` and `stop` (both or neither) stamped by the
 * runtime at the start and end of the cast kernels' own dispatch, so that
 * their elapsed time is the kernels' alone, whatever the stream waited for
 * before them.  No counterpart in the reference (it has no device cast);
 * used to measure the cast's HBM rate inside a training step. */
int sf_cast_f32_bf16_timed(const float* src, uint16_t* dst, size_t n,
                           sf_stream_t stream, sf_event_t start,
                           sf_event_t stop);

/* fp32 -> fp16 for units of dtype float16: IEEE round to nearest even with
 * subnormals, overflow to infinity, NaN -> quiet NaN (sign and the top 9
 * payload bits kept), dst[i] = rne_f16(src[i]) for i < n.  The cast of
 * layer_state.py:301 when the convert buffer has the config's dtype float16
 * (config.py:110-113, slide_fsdp.py:181-186): torch's CPU fp32 -> fp16
 * conversion, here in HBM.  The _timed variant stamps events as
 * sf_cast_f32_bf16_timed does. */
int sf_cast_f32_f16(const float* src, uint16_t* dst, size_t n,
                    sf_stream_t stream);
int sf_cast_f32_f16_timed(const float* src, uint16_t* dst, size_t n,
                          sf_stream_t stream, sf_event_t start,
                          sf_event_t stop);

/* Stage n fp32 values from pinned host memory into a bf16 device array:
 * dst[i] = rne(host_src[i]) (the rounding of sf_cast_f32_bf16).  The values
 * travel in pieces of workspace_elems (rounded down to a multiple of 8)
 * through the caller's device fp32 `workspace`: each piece is copied into
 * it by DMA and cast from it into dst, all in order on `stream`, so the
 * workspace may be reused once the stream has passed the call.  host_src
 * must be pinned host memory (SF_EINVAL otherwise: an asynchronous copy
 * needs it), dst and workspace device memory.  Replaces the reference's
 * staging of one unit, layer_state.py:299-314 (host cast of the flat master
 * into the pinned convert buffer, then a non_blocking bf16 copy on the H2D
 * stream), with the cast moved to the device. */
int sf_stage_f32_bf16(const float* host_src, uint16_t* dst, size_t n,
                      float* workspace, size_t workspace_elems,
                      sf_stream_t stream);

/* Elements (fp32) of the device scratch buffer of
 * sf_stage_f32_bf16_noalloc: 64 MiB on every device the library runs on,
 * held until the process ends. */
#define SF_STAGE_SCRATCH_ELEMS ((size_t)16 << 20)

/* sf_stage_f32_bf16 that allocates nothing: the pieces (chunk_elems fp32
 * elements; 0 selects SF_STAGE_SCRATCH_ELEMS, more is refused with
 * SF_ETOOBIG before anything is enqueued) go through a device buffer of the
 * library's own, one static array per device, whose address is looked up
 * (and one ordering event created) on the first call on each device.
 * `stream` must belong to the current device.  No hipMalloc, hipFree or
 * other allocating call is made after that first call.  Every call on a
 * device uses that device's one buffer, so the library orders the calls:
 * each call's stream first waits for the last cast of the previous call on
 * that device (an event recorded after it), then the call records the event
 * after its own last cast.  Calls on different streams are therefore
 * serialised on the device, in the order their host calls enter the
 * library.  No counterpart in the reference; for callers that cannot
 * allocate device memory (tight serving loops, harnesses that forbid
 * allocation). */
int sf_stage_f32_bf16_noalloc(const float* host_src, uint16_t* dst, size_t n,
                              size_t chunk_elems, sf_stream_t stream);

/* Timing events for sf_cast_f32_bf16_timed: create, destroy, and the
 * milliseconds between two completed events (a HIP status, e.g. not ready,
 * while either is pending).  No counterpart in the reference. */
int sf_event_create(sf_event_t* ev);
int sf_event_destroy(sf_event_t ev);
int sf_event_elapsed_ms(sf_event_t start, sf_event_t stop, float* ms);

/* The same cast over a table of segments (src: fp32, dst: bf16), for a
 * device layer buffer whose per-parameter views are not offset-identical
 * to the flat master.  The reference's views are offset-identical
 * (layer_state.py:246-250 and :318-320), where one sf_cast_f32_bf16 over
 * the whole layer is the same operation. */
int sf_cast_scatter_f32_bf16(const sf_seg* segs, int nsegs,
                             sf_stream_t stream);

/* ---------------------------------------------------------------------
 * Gradient and activation packing (libsf_hip.so)
 * ------------------------------------------------------------------- */

/* The segment-copy entry points below take max_workgroups: <= 0 launches
 * one workgroup per 8192-element tile (device-to-device work, all CUs);
 * a positive value caps the grid, each workgroup then striding over tiles.
 * A capped grid is meant for a destination in pinned host memory (the
 * device address from sf_host_device_pointer), where a few dozen
 * workgroups already saturate the host link and the remaining CUs stay
 * free for compute. */

/* Gather: for each segment k, copy segs[k].n 16-bit elements from
 * segs[k].src to dst + (sum of the n of segments before k).  segs[k].dst
 * is ignored.  Packs a layer's per-parameter bf16 gradients into one
 * contiguous buffer -- with dst in pinned host memory, straight into the
 * host staging slot, so the pack and the D2H are one kernel.  Replaces the
 * per-parameter grad views into the shared grad buffer that
 * layer_state.py:250 and :321-322 set up plus the D2H at
 * distributed_sync.py:353. */
int sf_pack_b16(const sf_seg* segs, int nsegs, uint16_t* dst,
                int max_workgroups, sf_stream_t stream);

/* Scatter, the inverse of sf_pack_b16: for each segment k, copy segs[k].n
 * elements from src + (sum of earlier n) to segs[k].dst.  segs[k].src is
 * ignored.  Restores packed checkpoint tensors (sliding_checkpoint.py:
 * 104-105) when they were packed from non-contiguous sources. */
int sf_unpack_b16(const uint16_t* src, const sf_seg* segs, int nsegs,
                  int max_workgroups, sf_stream_t stream);

/* General 16-bit segment copy: both addresses taken from each segment.
 * Also packs checkpoint tensors into their pinned host slots
 * (sliding_checkpoint.py:69-73). */
int sf_copy_segs_b16(const sf_seg* segs, int nsegs, int max_workgroups,
                     sf_stream_t stream);

/* dst[i] = value for i < n (16-bit elements), as a kernel rather than a
 * memset node so it is safe inside captured graphs (a GPU test replays a
 * captured fill and cast four times with eager work between).  Replaces
 * `_current_gpu_cache["grad"].zero_()`, layer_state.py:296-297. */
int sf_fill_b16(uint16_t* dst, size_t n, uint16_t value,
                sf_stream_t stream);

/* Row gather for a row-sparse embedding unit.  For t < ntok,
 * dst[t*row_len .. +row_len) = src row ids[t] of a [nrows, row_len] table,
 * rounded fp32 -> bf16 (RNE, NaN -> 0xFFFF) by the f32 variant, copied by the
 * b16 one.  src and dst may be device addresses of pinned host memory (the
 * forward reads only the batch's rows of the host master; the backward
 * writes only the batch's gradient rows to host).  An id outside
 * [0, nrows) gives a row of 0xFFFF and sets *bad = 1 (bad may be NULL).
 * max_workgroups > 0 caps the grid (host destinations).  Replaces the full
 * staging of the embedding unit (layer_state.py:296-314) for its forward
 * lookup (slide_fsdp.py:543-545, nn.Embedding) and the full gradient D2H
 * of that unit (layer_state.py:367-393). */
int sf_gather_rows_f32_bf16(const float* src, const int64_t* ids, size_t ntok,
                            size_t row_len, size_t nrows, uint16_t* dst,
                            uint32_t* bad, int max_workgroups,
                            sf_stream_t stream);
int sf_gather_rows_b16(const uint16_t* src, const int64_t* ids, size_t ntok,
                       size_t row_len, size_t nrows, uint16_t* dst,
                       uint32_t* bad, int max_workgroups, sf_stream_t stream);

/* ---------------------------------------------------------------------
 * Copies and pinned host memory (libsf_hip.so)
 * ------------------------------------------------------------------- */

#define SF_COPY_H2D 1
#define SF_COPY_D2H 2
#define SF_COPY_D2D 3

/* Asynchronous copy of `bytes` bytes on `stream`.  Host memory must be
 * pinned (sf_host_alloc) for the copy to be asynchronous.  Replaces the
 * non_blocking copies at distributed_sync.py:332 (params H2D),
 * distributed_sync.py:353 (grads D2H), sliding_checkpoint.py:73
 * (activation D2H) and sliding_checkpoint.py:105 (activation H2D). */
int sf_memcpy_async(void* dst, const void* src, size_t bytes, int kind,
                    sf_stream_t stream);

/* Exact-size pinned host allocation (no power-of-two rounding).  Replaces
 * `torch.empty(..., pin_memory=True)` for the fp32 flat masters
 * (layer_state.py:203-208), the shared grad and convert buffers
 * (slide_fsdp.py:174-186) and the activation slots (slide_fsdp.py:
 * 480-503). */
int sf_host_alloc(void** out, size_t bytes);
int sf_host_free(void* ptr);

/* Device-side address of pinned host memory, for kernels that read or
 * write host memory directly (hipHostGetDevicePointer). */
int sf_host_device_pointer(void* host_ptr, void** device_ptr);

/* ---------------------------------------------------------------------
 * SDMA device -> host copies (libsf_hip.so)
 *
 * A shader copy into host memory (hipMemcpyAsync's blit, or a pack kernel
 * with a host destination) slows HBM-bound kernels running beside it; an
 * SDMA engine does not.  These copies go through the ROCr runtime and are
 * NOT ordered with HIP streams: the caller must have completed the source
 * (e.g. synchronised an event on the host) before sf_dma_copy_d2h, and may
 * read the destination only after sf_dma_wait.  They replace the gradient
 * D2H of distributed_sync.py:353 (layer_state.py:367-381).
 * ------------------------------------------------------------------- */

/* Bind to the ROCr agents of HIP device `device` (once per process) and
 * pick the SDMA engine for device -> host copies: engine 3 if available,
 * else engine 2, else the runtime's choice.  HIP puts each of its own
 * host<->device copies on the first free engine (0, then 1, then 2); one
 * of them ordered after an event that has not fired holds its engine until
 * then, and a copy queued behind it waits as long.  One of engines 0-3
 * moves as much device -> host as two. */
int sf_dma_init(int device);

/* Override the engines (bit e = SDMA engine e; 0 = runtime's choice). */
int sf_dma_set_engines(uint32_t engine_mask);
int sf_dma_get_engines(uint32_t* engine_mask);

/* Route around held engines: mode 0 no (the default), 1 onto free engines
 * 0-3, 2 also onto free engines from 4 up when none of 0-3 is free.  Each
 * sf_dma_copy_d2h then asks the runtime which engines are free; an engine
 * of the selected set that is busy while none of this library's copies is
 * pending on it is held by another client (a HIP copy ordered after an
 * event that has not fired holds its engine until then), and the copies go
 * to free engines in its place (engines from 4 up: twice as many, they are
 * slower for host copies).  SF_EINVAL for another mode.  No reference
 * counterpart (its D2H is a torch copy on a stream, layer_state.py:367-393). */
int sf_dma_set_avoid_held(int mode);

/* The engine choice of sf_dma_copy_d2h as a pure function: from the
 * selected engines `preferred`, the runtime's free engines `avail` and the
 * engines with copies of this library pending `ours`, the engines to use
 * under `mode` (see sf_dma_set_avoid_held).  No GPU access; for tests. */
uint32_t sf_dma_choose_engines(uint32_t preferred, uint32_t avail, uint32_t ours, int mode);

/* For each segment, copy segs[k].n BYTES from device address segs[k].src
 * to pinned host address segs[k].dst.  Segments of 4 MiB or more are split
 * evenly over the selected engines, others go round-robin.  One completion
 * handle per issued copy is written to signals (at most max_signals);
 * *nsignals receives their number.  Every segment is checked before the
 * first copy is issued.  If a later step fails (SF_ETOOMANY, or a ROCr call
 * as SF_EDMA_BASE + status), the copies issued before it still run:
 * *nsignals and signals[] then describe them, and the caller must wait for
 * them (sf_dma_wait) before reusing the destinations or freeing the
 * sources. */
int sf_dma_copy_d2h(const sf_seg* segs, int nsegs, uint64_t* signals,
                    int max_signals, int* nsignals);

/* Wait until every handle has completed, then release them.  timeout_ns
 * bounds the wait (0: no limit); when it passes with a copy still pending,
 * SF_ETIMEDOUT is returned and no handle is released (each stays valid for
 * a later sf_dma_query or sf_dma_wait; the copies keep running).  The wait
 * polls the completion signals with 50 us sleeps.  If start_ns and end_ns
 * are non-null and timing is enabled, they receive the earliest start and
 * the latest end of the copies, in ns of the HSA system clock (both 0 when
 * timing is off). */
int sf_dma_wait(const uint64_t* signals, int nsignals, uint64_t timeout_ns,
                uint64_t* start_ns, uint64_t* end_ns);

/* Non-blocking completion test of copies started by sf_dma_copy_d2h:
 * *done = 1 when every signal has completed, else 0.  The signals stay
 * valid (sf_dma_wait still has to be called to release them).  No
 * reference counterpart (the reference's D2H is a blocking torch copy,
 * layer_state.py:367-393); used to run host updates as their copies land. */
int sf_dma_query(const uint64_t* signals, int nsignals, int* done);

/* Record start/end times of later copies (1) or stop (0). */
int sf_dma_enable_timing(int on);

/* The HSA system clock now, in ns: the clock of the copy times of
 * sf_dma_wait, so a caller can place other timestamps (HIP events, anchored
 * once) on the same timeline.  No reference counterpart; measurement only. */
int sf_dma_clock_ns(uint64_t* ns);

/* ---------------------------------------------------------------------
 * Host AdamW (libsf_cpu.so)
 * ------------------------------------------------------------------- */

#define SF_DTYPE_F32 0
#define SF_DTYPE_BF16 1
#define SF_DTYPE_F16 2

/* Scalars of one update, precomputed by the caller. */
typedef struct sf_adam_hparams {
    float beta1;
    float beta2;
    float eps;
    float weight_decay;
    float step_size;        /* -lr / bias_correction1                   */
    float bias_correction2; /* 1 / sqrt(1 - beta2^t), or 1 if disabled  */
    float lr;
    int adamw_mode;         /* 1: decoupled decay; 0: L2 into the grad  */
} sf_adam_hparams;

/* Stateless AdamW over n elements: fp32 params and moments updated in
 * place, grads read as g_dtype (SF_DTYPE_F32, SF_DTYPE_BF16 or
 * SF_DTYPE_F16; 16-bit grads are widened exactly, so the result equals the
 * fp32 call on `grad.float()`).
 * Per-element operation order follows Adam_Optimizer::Step_AVX,
 * optimizer/layer_adam/csrc/cpu_adam.h:143-192. */
int sf_cpu_adam_step(float* params, const void* grads, int g_dtype,
                     float* exp_avg, float* exp_avg_sq, size_t n,
                     const sf_adam_hparams* hp);

/* sf_cpu_adam_step, also writing params_bf16[i] = rne_bf16(params[i]) after
 * the update (same rounding and NaN rule as sf_cast_f32_bf16).  Feeds the
 * optional bf16 host-to-device mode: the host keeps a bf16 copy of every
 * master current, so only 2 bytes per parameter cross the host link, as in
 * the reference (layer_state.py:301 casts on the host before the H2D). */
int sf_cpu_adam_step_cast(float* params, const void* grads, int g_dtype,
                          float* exp_avg, float* exp_avg_sq,
                          uint16_t* params_bf16, size_t n,
                          const sf_adam_hparams* hp);

/* Host fp32 -> bf16 cast with the same rounding (OpenMP + AVX-512). */
int sf_cpu_cast_f32_bf16(const float* src, uint16_t* dst, size_t n);

/* Stateful interface with the reference's pybind11 `cpu_adam` module
 * semantics (optimizer/layer_adam/csrc/cpu_adam.cpp:8-13):
 *   create_adam  -> sf_adam_create   (cpu_adam_impl.cpp:89-127)
 *   adam_update  -> sf_adam_update   (cpu_adam_impl.cpp:211-237)
 *   destroy_adam -> sf_adam_destroy  (cpu_adam_impl.cpp:239-244)
 * sf_adam_update keeps the reference's per-optimizer beta^t running
 * state (cpu_adam.h:57-89).  Unlike the reference, an unknown id returns
 * SF_ENOOPT and the registry is locked. */
int sf_adam_create(int optimizer_id, float alpha, float beta1, float beta2,
                   float eps, float weight_decay, int adamw_mode,
                   int should_log);
int sf_adam_update(int optimizer_id, size_t step, float lr, float beta1,
                   float beta2, float eps, float weight_decay,
                   int bias_correction, float* params, const void* grads,
                   int g_dtype, float* exp_avg, float* exp_avg_sq, size_t n);
int sf_adam_destroy(int optimizer_id);

/* sf_adam_update that also writes the bf16 copy of the updated params
 * (params_bf16 may be NULL). */
int sf_adam_update_cast(int optimizer_id, size_t step, float lr, float beta1,
                        float beta2, float eps, float weight_decay,
                        int bias_correction, float* params, const void* grads,
                        int g_dtype, float* exp_avg, float* exp_avg_sq,
                        uint16_t* params_bf16, size_t n);

/* sf_adam_update_cast over a [n_rows, row_len] tensor whose gradient is
 * zero except in some rows: row r takes its gradient from row row_slot[r]
 * of grads ([n_grad_rows, row_len], g_dtype), zeros when row_slot[r] is
 * SF_ROW_ZERO, and is left as it is when row_slot[r] is SF_ROW_SKIP (so an
 * update can be split over rows: the rows of one call skipped by the other).
 * Other negative values are an error.  Every element gets exactly the dense
 * update (row_len must be a multiple of 16, so no element falls in the
 * scalar tail).  Replaces adam_update on the embedding unit's dense
 * `grad.float()` (layer_adam.py:404) when only the batch's rows were
 * offloaded. */
#define SF_ROW_ZERO (-1)
#define SF_ROW_SKIP (-2)
int sf_adam_update_rows(int optimizer_id, size_t step, float lr, float beta1,
                        float beta2, float eps, float weight_decay,
                        int bias_correction, float* params, float* exp_avg,
                        float* exp_avg_sq, uint16_t* params_bf16,
                        size_t n_rows, size_t row_len, const int64_t* row_slot,
                        const void* grads, size_t n_grad_rows, int g_dtype);

/* Scalars of one update of step `step` as the reference's stateful call
 * sequence yields them (Adam_Optimizer::IncrementStep and its bias
 * corrections, cpu_adam.h:57-89) when every unit is stepped once per step,
 * last unit first, with at least two calls per step: first_of_step = 1 for
 * the first call of the step (the last unit's first parameter), 0 for every
 * other.  No optimizer state is read or written, so a caller that updates
 * units in another order still gets the reference's bits.  No reference
 * counterpart (the reference's order is fixed: updates run first in, first
 * out, slide_fsdp.py:163). */
int sf_adam_hparams_in_order(size_t step, float lr, float beta1, float beta2,
                             float eps, float weight_decay, int bias_correction,
                             int adamw_mode, int first_of_step,
                             sf_adam_hparams* hp);

/* sf_adam_update_rows with caller-given scalars and no optimizer state. */
int sf_cpu_adam_step_rows(float* params, float* exp_avg, float* exp_avg_sq,
                          uint16_t* params_bf16, size_t n_rows, size_t row_len,
                          const int64_t* row_slot, const void* grads,
                          size_t n_grad_rows, int g_dtype,
                          const sf_adam_hparams* hp);

/* OpenMP team size used by the host AdamW (<= 0: library default). */
int sf_cpu_set_threads(int nthreads);
/* 1 if the AVX-512 path is used on this host, 0 for the portable path. */
int sf_cpu_has_avx512(void);

/* ---------------------------------------------------------------------
 * Storage offload engine (libsf_cpu.so)
 *
 * Moves host buffers to and from files: checkpointed activations (through
 * pinned bounce slots) and LayerAdam moments.  Replaces the reference's two
 * storage back ends, neither of which exists for ROCm:
 *   kvikio CuFile raw_write_async / raw_read_async (GPUDirect Storage;
 *     sliding_checkpoint.py:133-202)
 *   tensornvme DiskOffloader async_write / async_read / sync_*_events
 *     (optimizer/layer_adam/layer_adam.py:89-103, 197-244)
 * A request is cut into chunk_bytes pieces moved by n_threads workers with
 * pread/pwrite.  Files are opened with O_DIRECT where the file system allows
 * it; then the buffer address, the size and the file offset of a request
 * must be multiples of SF_IO_ALIGN (SF_EALIGN otherwise).  Pinned host
 * memory from hipHostMalloc cannot be pinned again by the kernel for direct
 * I/O; chunks of such buffers are copied through a per-worker staging buffer.
 * ------------------------------------------------------------------- */

#define SF_IO_READ 0
#define SF_IO_WRITE 1
#define SF_IO_ALIGN 4096

typedef struct sf_io sf_io;

/* Start an engine with n_threads workers (1..256); chunk_bytes 0 selects
 * 8 MiB, other values are rounded up to SF_IO_ALIGN. */
int sf_io_create(int n_threads, size_t chunk_bytes, sf_io** out);
/* Finish every queued request, stop the workers and free the engine. */
int sf_io_destroy(sf_io* io);

/* Open (creating) a file for reading and writing.  direct = 1 asks for
 * O_DIRECT; where the file system refuses it the file is opened buffered and
 * *direct_out (if non-null) is 0.  unlink_now = 1 removes the name at once,
 * so the space is returned when the descriptor is closed or the process
 * ends.  (kvikio.CuFile(path, "w"/"r"), sliding_checkpoint.py:148, 179;
 * DiskOffloader(dir, ...), layer_adam.py:98.) */
int sf_io_open(const char* path, int direct, int unlink_now, int* fd,
               int* direct_out);
/* Extend the file to at least `bytes` (unwritten ranges read as zeros). */
int sf_io_reserve(int fd, uint64_t bytes);
int sf_io_close(int fd);

/* Queue a read (SF_IO_READ: file -> buf) or write (SF_IO_WRITE: buf -> file)
 * of `bytes` at file `offset`; *ticket names the request.  The buffer must
 * stay valid until the request completes.  (raw_write_async /
 * raw_read_async, sliding_checkpoint.py:149, 181; async_write / async_read,
 * layer_adam.py:205-207, 216-218.) */
int sf_io_submit(sf_io* io, int fd, int op, void* buf, size_t bytes,
                 uint64_t offset, uint64_t* ticket);
/* Non-blocking: *done = 1 once the request completed, and then the return
 * value is its status (0, or SF_EIO_BASE + errno of the first failed chunk).
 * The ticket stays valid. */
int sf_io_query(sf_io* io, uint64_t ticket, int* done);
/* Block until the request completed, release the ticket and return its
 * status; submit_ns / done_ns (if non-null) receive its CLOCK_MONOTONIC
 * submit and completion times.  (check_bytes_done / sync_*_events,
 * sliding_checkpoint.py:177, 190; layer_adam.py:227, 236.) */
int sf_io_wait(sf_io* io, uint64_t ticket, uint64_t* submit_ns,
               uint64_t* done_ns);
/* Bytes read and written by completed requests, the time during which at
 * least one request was in flight (ns), and the bytes that went through a
 * worker's staging buffer because the kernel could not pin the caller's
 * pages for direct I/O (memory from hipHostMalloc). */
int sf_io_stats(sf_io* io, uint64_t* bytes_read, uint64_t* bytes_written,
                uint64_t* busy_ns, uint64_t* bytes_staged);

#ifdef __cplusplus
}
#endif

#endif /* SLIDEFSDP_H */
