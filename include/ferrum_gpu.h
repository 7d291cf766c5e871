/*
 * ferrum_gpu.h -- C ABI of the MI355X-native ferrum-gpu FFT backend.
 *
 * Plain pointers and sizes only.  Every function returns an int status
 * (FG_OK = 0, negative on failure) and leaves a thread-local message in
 * fg_last_error().  Complex data is interleaved complex64 ([re, im] f32
 * pairs), the layout of the reference's Complex32
 * (crates/ferrum-gpu-fft/src/complex.rs:10-53) and of numpy complex64.
 *
 * Each declaration cites the reference interface it replaces (paths relative
 * to the reference repository root).
 */
#ifndef FERRUM_GPU_H
#define FERRUM_GPU_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__)
#define FG_API __attribute__((visibility("default")))
#else
#define FG_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- status */

/* Error variants of crates/ferrum-gpu-cuda/src/error.rs:9-34 and
 * crates/ferrum-gpu-core/src/error.rs:11-34, plus argument/memory errors the
 * Python layer reports as ValueError (crates/ferrum-gpu-py/src/lib.rs:455-477). */
#define FG_OK 0
#define FG_ERR_INVALID_ARGUMENT (-1)
#define FG_ERR_DRIVER (-2)           /* HIP runtime error (CudaBackendError::Driver) */
#define FG_ERR_BACKEND_MISMATCH (-3) /* FerrumGpuError::BackendMismatch */
#define FG_ERR_KERNEL_NOT_FOUND (-4) /* FerrumGpuError::KernelNotFound */
#define FG_ERR_TARGET_MISMATCH (-5)  /* code object built for another gfx target */
#define FG_ERR_OUT_OF_MEMORY (-6)
#define FG_ERR_NO_DEVICE (-7)
#define FG_ERR_INTERNAL (-8)

/* BackendId (crates/ferrum-gpu-core/src/artifact.rs:13-36) with Hip added. */
#define FG_BACKEND_CUDA 1
#define FG_BACKEND_VULKAN 2
#define FG_BACKEND_HIP 3

/* Direction (crates/ferrum-gpu-core/src/dim.rs:52-64). */
#define FG_FORWARD 1
#define FG_INVERSE (-1)

/* Thread-local text of the last failure on this thread ("" if none). */
FG_API const char *fg_last_error(void);
/* Crate version string, "0.3.0" (crates/ferrum-gpu-py/src/lib.rs:420-423). */
FG_API const char *fg_version(void);
/* Backend::id() (crates/ferrum-gpu-core/src/backend.rs:27): FG_BACKEND_HIP. */
FG_API int fg_backend_id(void);

/* ---------------------------------------------------------------- device */

typedef struct fg_device *fg_device_t;
typedef struct fg_module *fg_module_t;
typedef struct fg_kernel *fg_kernel_t;
typedef struct fg_event *fg_event_t;
typedef void *fg_stream_t; /* a hipStream_t */

/* Number of visible GPUs (0 on a machine without one). */
FG_API int fg_device_count(int *count);
/* Device::new(ordinal) (crates/ferrum-gpu/src/lib.rs:22-40,
 * crates/ferrum-gpu-py/src/lib.rs:400-408): select the GPU, create its default
 * stream and load the FFT code object into the device's module cache. */
FG_API int fg_device_open(int ordinal, fg_device_t *out);
/* Drop of Device: waits for the default stream, frees what the device owns.
 * Refused (FG_ERR_INVALID_ARGUMENT) while plans or captured graphs made on the
 * device are alive: destroy them first. */
FG_API int fg_device_close(fg_device_t dev);
/* Device::sync (crates/ferrum-gpu/src/device.rs:36-38, py lib.rs:410-416). */
FG_API int fg_device_sync(fg_device_t dev);
/* Backend::default_stream (crates/ferrum-gpu-core/src/backend.rs:73). */
FG_API int fg_device_default_stream(fg_device_t dev, fg_stream_t *out);
/* Name ("gfx950"...), compute units and total memory of the device. */
FG_API int fg_device_info(fg_device_t dev, char *arch, size_t arch_cap, int *cu_count,
                   size_t *total_mem_bytes, int *clock_khz);

/* --------------------------------------------------------------- buffers */

/* Backend::alloc_zeros (backend.rs:30-33): synchronous, zero-filled. */
FG_API int fg_alloc_zeros(fg_device_t dev, size_t bytes, void **dptr);
/* Drop of CudaBuffer (crates/ferrum-gpu-cuda/src/buffer.rs:45-56): waits for
 * the device's default stream, then frees. */
FG_API int fg_free(fg_device_t dev, void *dptr);
/* Backend::copy_h2d / copy_d2h (backend.rs:35-47): synchronous. */
FG_API int fg_copy_h2d(fg_device_t dev, void *dst, const void *src, size_t bytes);
FG_API int fg_copy_d2h(fg_device_t dev, void *dst, const void *src, size_t bytes);
/* Stream-ordered variants (the async copies the north star adds). */
FG_API int fg_copy_h2d_async(fg_device_t dev, void *dst, const void *src, size_t bytes,
                      fg_stream_t stream);
FG_API int fg_copy_d2h_async(fg_device_t dev, void *dst, const void *src, size_t bytes,
                      fg_stream_t stream);
FG_API int fg_copy_d2d_async(fg_device_t dev, void *dst, const void *src, size_t bytes,
                      fg_stream_t stream);

/* ------------------------------------------------------ modules, launch */

/* Backend::load_module (backend.rs:50-53, crates/ferrum-gpu-cuda/src/backend_impl.rs:75-87):
 * loads a gfx950 code object; backend_id must be FG_BACKEND_HIP, otherwise
 * FG_ERR_BACKEND_MISMATCH. */
FG_API int fg_module_load(fg_device_t dev, int backend_id, const void *image, size_t size,
                   fg_module_t *out);
FG_API int fg_module_unload(fg_module_t mod);
/* The FFT module the device loaded at open (owned by the device). */
FG_API int fg_device_fft_module(fg_device_t dev, fg_module_t *out);
/* Backend::get_kernel (backend.rs:56-59): FG_ERR_KERNEL_NOT_FOUND if absent. */
FG_API int fg_kernel_get(fg_module_t mod, const char *name, fg_kernel_t *out);
/* Backend::launch (backend.rs:62-70): args[i] points at the i-th kernel
 * argument's bytes (device pointers and scalars alike). stream NULL = default. */
FG_API int fg_launch(fg_device_t dev, fg_stream_t stream, fg_kernel_t kernel, const uint32_t grid[3],
              const uint32_t block[3], uint32_t shared_bytes, void **args);

/* --------------------------------------------------------- streams/events */

FG_API int fg_stream_create(fg_device_t dev, fg_stream_t *out); /* default priority */
FG_API int fg_stream_destroy(fg_device_t dev, fg_stream_t stream);
/* Backend::sync_stream (backend.rs:75-76). NULL = the device default stream. */
FG_API int fg_stream_sync(fg_device_t dev, fg_stream_t stream);
FG_API int fg_event_create(fg_device_t dev, fg_event_t *out);
FG_API int fg_event_destroy(fg_event_t ev);
/* Records the event on `stream`; NULL = the default stream of the device the
 * event was created on (the stream fg_fft_exec and the copies use for NULL). */
FG_API int fg_event_record(fg_event_t ev, fg_stream_t stream);
FG_API int fg_event_sync(fg_event_t ev);
FG_API int fg_event_elapsed_ms(fg_event_t start, fg_event_t end, float *ms);

/* -------------------------------------------------------------------- FFT */

typedef struct fg_fft_plan *fg_fft_plan_t;

/* Plan::new(log_n, batch, normalize) (crates/ferrum-gpu-fft/src/plan.rs:57-68)
 * on a device: builds the twiddle tables in HBM once and picks the kernel(s).
 * log_n in [2, 24] (the reference stops at 12, plan.rs:58).  batch >= 1. */
FG_API int fg_fft_plan_1d(fg_device_t dev, uint32_t log_n, size_t batch, fg_fft_plan_t *out);
/* Plan2D::new(log_n, normalize) (plan.rs:111-119) for `batch` square N x N
 * row-major images; log_n in [4, 12] (py lib.rs:537-541). */
FG_API int fg_fft_plan_2d(fg_device_t dev, uint32_t log_n, size_t batch, fg_fft_plan_t *out);
FG_API int fg_fft_plan_destroy(fg_fft_plan_t plan);
/* Device-resident execution, stream-ordered and asynchronous: the kernel
 * launch of the host runner (py lib.rs:142-233, 325-358) with the inverse's
 * conjugation and 1/N (1/(N*N) for 2D) scaling done inside the kernels.
 * d_in and d_out each hold batch*N (2D: batch*N*N) complex64, 8-byte aligned;
 * they may be equal (in place) but must not otherwise overlap.
 * direction: FG_FORWARD or FG_INVERSE.  stream NULL = device default stream.
 * A multi-launch plan (1D N > 32768, 2D images above 16384 points) keeps one
 * workspace (two for two-stream plans, fg_fft_plan_streams) and one
 * split-layout staging buffer: executions of one plan must be ordered, one
 * stream at a time; run concurrent work on separate plans. */
FG_API int fg_fft_exec(fg_fft_plan_t plan, const void *d_in, void *d_out, int direction, int normalize,
                fg_stream_t stream);
/* fg_fft_exec that also records events[i] right after launch i (nevents must
 * equal the plan's launch count); no synchronisation.  Launch i's duration is
 * the time from the previous event on its stream (the caller's start event,
 * or events[i-1]) to events[i]; on a two-stream plan (fg_fft_plan_streams)
 * the launches of odd chunks run, and stamp their events, on the plan's
 * second stream, whose first launch starts when the caller's stream reaches
 * the call.  For per-kernel timing
 * in benchmarks: the reference's bench brackets its single launch with an
 * event pair (crates/ferrum-gpu-bench/src/lib.rs:163-198); here each event is
 * stamped by its launch's dispatch (no marker packet between back-to-back
 * launches), so the timed sequence runs as fg_fft_exec would. */
FG_API int fg_fft_exec_events(fg_fft_plan_t plan, const void *d_in, void *d_out, int direction,
                              int normalize, fg_stream_t stream, fg_event_t *events, int nevents);
/* HIP graphs of plan executions.  No counterpart in the reference, whose host
 * runner submits every kernel from the host on each call
 * (crates/ferrum-gpu-py/src/lib.rs:142-233); for callers whose loop is bound
 * by launch latency (small batches, serving loops).
 * fg_fft_graph_create captures `reps` back-to-back fg_fft_exec(plan, d_in,
 * d_out, direction, normalize) into one executable graph (reps * launches
 * kernel nodes, at most 65536; kernel launches only: no memset, copy or
 * allocation nodes).  Nothing runs at creation.  The graph keeps d_in, d_out
 * and the plan's tables and workspace by address: the buffers must stay
 * allocated while it is used, and fg_fft_plan_destroy refuses a plan that
 * still has graphs.  fg_graph_launch enqueues one replay on `stream` (NULL =
 * the device default stream), stream-ordered and asynchronous; replays on one
 * stream run one after another, and replays that overlap on different streams
 * race on the same buffers. */
typedef struct fg_graph *fg_graph_t;
FG_API int fg_fft_graph_create(fg_fft_plan_t plan, const void *d_in, void *d_out, int direction,
                               int normalize, int reps, fg_graph_t *out);
FG_API int fg_graph_launch(fg_graph_t graph, fg_stream_t stream);
/* General capture: fg_graph_capture_begin returns a new stream of the device
 * in thread-local capture mode; stream-ordered fg_* calls made on it from the
 * calling thread (fg_fft_exec, the elementwise kernels, fg_transpose_c64, ...)
 * are recorded instead of run, and fg_graph_capture_end turns them into one
 * graph and destroys the stream.  Make calls that allocate (the first
 * fg_fft_exec_split of a multi-launch plan, which refuses to run on a
 * capturing stream) once before capturing.  The caller
 * keeps every plan and buffer the recorded calls use alive while the graph is
 * launched.  fg_graph_capture_end must be called once per begin, also after
 * a failed call. */
FG_API int fg_graph_capture_begin(fg_device_t dev, fg_stream_t *capture_stream);
FG_API int fg_graph_capture_end(fg_device_t dev, fg_stream_t capture_stream, fg_graph_t *out);
/* Number of nodes in the captured graph. */
FG_API int fg_graph_node_count(fg_graph_t graph, size_t *nodes);
FG_API int fg_graph_destroy(fg_graph_t graph);
/* Chunked execution of multi-launch plans (1D N > 32768, 2D images above
 * 16384 points).  No
 * counterpart in the reference, whose GPU path has no multi-pass plans
 * (crates/ferrum-gpu-fft/src/plan.rs:58).  Such a plan runs all of its passes
 * over one chunk (whole transforms or images) before the next, keeping the
 * chunk's intermediate array cached (in the 256 MB Infinity Cache) instead of
 * moving it through HBM.  `bytes` bounds the chunks in flight at once: plans
 * that run two chunks at a time (fg_fft_plan_streams) take chunks of at most
 * bytes / 2 when a transform fits that (else one chunk at a time, of at most
 * `bytes`), the others chunks of at most `bytes`.  The limit applies to plans
 * created afterwards, process-wide; 0 disables chunking (one chunk of the
 * whole batch, every pass streaming).  Default: FERRUM_GPU_CHUNK_MIB from the
 * environment when the library loads, else 256 MiB. */
FG_API int fg_fft_set_chunk_bytes(size_t bytes);
FG_API int fg_fft_get_chunk_bytes(size_t *bytes);
/* How a plan executes: passes per chunk, transforms (2D: images) per chunk,
 * number of chunks (launches = passes * chunks), and whether intermediates
 * are kept cached (1) or every pass streams (0). */
FG_API int fg_fft_plan_chunking(fg_fft_plan_t plan, int *passes, size_t *units_per_chunk, int *chunks,
                                int *cached);
/* Streams an execution runs on: 1, or 2 for multi-pass 1D plans of two or
 * more chunks, which run the odd chunks (launches passes*c .. passes*c +
 * passes - 1 of chunk c) with a second workspace on the device's chunk
 * stream (one per device, shared by every two-stream plan on it), forked
 * from the caller's stream when the execution starts and joined back to it
 * when it ends (so work enqueued on the caller's stream afterwards sees the
 * whole output).  On a capturing stream every chunk runs on the captured
 * stream.  The overlap of the two chunks needs the chunk stream on a
 * hardware queue of its own (HIP gives a process GPU_MAX_HW_QUEUES = 4 by
 * default).  No counterpart in the reference (one stream per call,
 * crates/ferrum-gpu-py/src/lib.rs:142-233). */
FG_API int fg_fft_plan_streams(fg_fft_plan_t plan, int *streams);
/* Runs a plan's chunks on one stream (streams = 1) or, for a plan that
 * fg_fft_plan_streams reported at 2 when it was created, on two again
 * (streams = 2; FG_ERR_INVALID_ARGUMENT for other plans or values).  Same
 * results bit for bit either way; no execution of the plan may be in flight
 * while it changes.  For callers whose own streams already occupy the
 * hardware queues, and for timing each pass on its own.  No counterpart in
 * the reference. */
FG_API int fg_fft_plan_set_streams(fg_fft_plan_t plan, int streams);
/* Kernel name of launch `index` of an execution out of place (d_in != d_out).
 * 2D plans of 2048 or 4096 rows of 1024 .. 4096 columns run other kernels in
 * place (fg_fft_n<log_cols> rows, then column tiles of all the rows), as many
 * launches: fg_fft_plan_kernel_in_place names those.  The two forms agree to
 * rounding, not bit for bit.  A plan's launches are passes * chunks; a batch
 * beyond one launch's 2^32 - 1 work-items (single-pass plans too) runs in
 * several chunks rather than being refused or truncated. */
FG_API int fg_fft_plan_kernel(fg_fft_plan_t plan, int index, char *name, size_t cap);
FG_API int fg_fft_plan_kernel_in_place(fg_fft_plan_t plan, int index, char *name, size_t cap);
/* Number of kernel launches per execution and the name of the kernel that
 * moves the most bytes (what the bench times and profiles). */
FG_API int fg_fft_plan_describe(fg_fft_plan_t plan, int *launches, char *main_kernel, size_t cap,
                         size_t *workspace_bytes);

/* Host-memory convenience path behind ferrum_gpu.fft.fft_1d_c2c_pow2
 * (crates/ferrum-gpu-py/src/lib.rs:445-504 -> run_fft_flat_with_device,
 * lib.rs:86-250): validate, copy in, execute, copy out, synchronous.
 * dev NULL uses a process-wide device 0 (the one-shot path, lib.rs:254-264).
 * total_complex must be a positive multiple of 2^log_n; log_n in [2, 24]. */
FG_API int fg_fft_1d_c2c_pow2_host(fg_device_t dev, const float *in, float *out, size_t total_complex,
                            uint32_t log_n, int direction, int normalize);
/* Behind ferrum_gpu.fft.fft_2d_c2c_pow2 (py lib.rs:527-588 -> run_fft_2d_flat,
 * lib.rs:273-375): `batch` images of N x N; log_n in [4, 12]. */
FG_API int fg_fft_2d_c2c_pow2_host(fg_device_t dev, const float *in, float *out, uint32_t log_n,
                            size_t batch, int direction, int normalize);

/* Non-square 2D (general power-of-two images, beyond Plan2D's square ones,
 * crates/ferrum-gpu-fft/src/plan.rs:98-135): `batch` row-major images of
 * 2^log_rows x 2^log_cols, each log in [4, 12]; normalize scales the inverse
 * by 1/(rows*cols). */
FG_API int fg_fft_plan_2d_rect(fg_device_t dev, uint32_t log_rows, uint32_t log_cols, size_t batch,
                               fg_fft_plan_t *out);
FG_API int fg_fft_2d_rect_host(fg_device_t dev, const float *in, float *out, uint32_t log_rows,
                               uint32_t log_cols, size_t batch, int direction, int normalize);
/* Tiled transpose out[b][c][r] = in[b][r][c] of `batch` rows x cols complex64
 * matrices on the device (the reference's transpose_complex_pow2 kernel,
 * crates/ferrum-gpu-fft-kernels/src/kernels_body.rs:763-805, for any shape);
 * in and out must not alias.  Stream-ordered, asynchronous. */
FG_API int fg_transpose_c64(fg_device_t dev, const void *d_in, void *d_out, uint32_t rows, uint32_t cols,
                            size_t batch, fg_stream_t stream);

/* Split layout (structure of arrays): real and imaginary parts in two f32
 * arrays of batch * elements each, transform f at element offset f * elements
 * (the reference's fft_c2c_{256_r16s,1024,4096_4step_reg}_split kernels,
 * crates/ferrum-gpu-fft-kernels/src/kernels_body.rs:509-626, 986-1130,
 * 1463-1610, for every plan).  Same results as fg_fft_exec on the interleaved
 * data; multi-launch plans run that execution in place on their staging
 * buffer, so for 2D plans of 2048 / 4096 rows of 1024 .. 4096 columns (whose
 * in-place execution differs, fg_fft_plan_kernel_in_place) the results equal
 * an in-place fg_fft_exec bit for bit and an out-of-place one to rounding.  Each array 4-byte aligned (FG_ERR_INVALID_ARGUMENT otherwise);
 * d_out_re / d_out_im may equal d_in_re / d_in_im; no other overlap.
 * Single-pass plans (1D, N <= 32768; 2D images of up to 16384 points) run one
 * launch; other plans stage through an interleaved buffer the plan allocates
 * at its first split call (synchronously: that first call is refused with
 * FG_ERR_INVALID_ARGUMENT, before any allocation, when `stream` is being
 * captured).
 * Stream-ordered, asynchronous. */
FG_API int fg_fft_exec_split(fg_fft_plan_t plan, const void *d_in_re, const void *d_in_im,
                             void *d_out_re, void *d_out_im, int direction, int normalize,
                             fg_stream_t stream);

/* fg_fft_exec_split that allocates nothing, on any call.  No counterpart in
 * the reference; it is for callers that cannot allocate device memory: code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  Multi-launch plans stage through a fixed device scratch area
 * of 64 MiB (67108864 bytes) that the library holds on each GPU it opens,
 * from fg_device_open until the process ends, instead of the plan's lazily
 * allocated buffer; a plan whose batch needs more staging (8 bytes per
 * element of batch * elements) is refused with FG_ERR_INVALID_ARGUMENT.
 * Single-pass plans need no staging and run as fg_fft_exec_split does.
 * Same results as fg_fft_exec_split, bit for bit (so, for the 2D plans named
 * there, the in-place interleaved execution's bits).  All callers on one GPU
 * share its scratch area, which keeps the last call's contents.  Outside
 * stream capture, calls that stage through it run one after another on the
 * GPU in the order they were made (each waits, on its stream, for an event
 * the previous one recorded after its last launch; the event is created at
 * fg_device_open), whatever streams or threads make them.  Captured calls
 * cannot wait for work outside their capture: graphs replayed so that they
 * overlap in time each other or other calls on one GPU race.
 * Stream-ordered, asynchronous. */
FG_API int fg_fft_exec_split_noalloc(fg_fft_plan_t plan, const void *d_in_re, const void *d_in_im,
                                     void *d_out_re, void *d_out_im, int direction, int normalize,
                                     fg_stream_t stream);

/* Elementwise kernels over n complex elements (kernels_body.rs:1612-1672).
 * Products are evaluated as re = ar*br - ai*bi, im = ar*bi + ai*br in f32
 * without fused multiply-add, like the reference.  Any alignment of complex64
 * / f32 data; 16-byte-aligned pointers take 16-byte accesses.  An output may
 * be the same array as an input of the same part; other overlaps are
 * rejected.  Stream-ordered, asynchronous. */
/* out = a * b, interleaved complex64 (cmul_interleaved, :1612-1627). */
FG_API int fg_cmul_c64(fg_device_t dev, const void *d_a, const void *d_b, void *d_out, size_t n,
                       fg_stream_t stream);
/* (o_re, o_im) = (a_re, a_im) * (b_re, b_im), split layout (cmul_split, :1629-1645). */
FG_API int fg_cmul_split(fg_device_t dev, const void *d_a_re, const void *d_a_im, const void *d_b_re,
                         const void *d_b_im, void *d_o_re, void *d_o_im, size_t n, fg_stream_t stream);
/* re[i], im[i] = in[i] (deinterleave, :1647-1659). */
FG_API int fg_deinterleave_c64(fg_device_t dev, const void *d_in, void *d_re, void *d_im, size_t n,
                               fg_stream_t stream);
/* out[i] = (re[i], im[i]) (interleave, :1661-1671). */
FG_API int fg_interleave_c64(fg_device_t dev, const void *d_re, const void *d_im, void *d_out, size_t n,
                             fg_stream_t stream);

/* Seeded synthetic data: n complex64 values written to d_out (8-byte aligned),
 * the same array for a given seed on any device, and equal to the CPU
 * restatement in oracle/ (uniform: bit for bit).  Float j of the output
 * (2i: real part of element i, 2i+1: imaginary part) uses the splitmix64
 * output z(j) for the state seed + (j+1) * 0x9E3779B97F4A7C15:
 *   uniform: (z(j) >> 40) * 2^-23 - 1, exactly representable, in [-1, 1);
 *   normal:  Box-Muller in f64 on (z(2i), z(2i+1)), rounded to f32.
 * The input generator the benchmark's configurations name ("seed = config
 * index"); it replaces the reference's per-example input loops
 * (e.g. examples/fft-1d-c2c/src/main.rs:131).  Stream-ordered, asynchronous. */
FG_API int fg_fill_uniform_c64(fg_device_t dev, void *d_out, size_t n, uint64_t seed,
                               fg_stream_t stream);
FG_API int fg_fill_normal_c64(fg_device_t dev, void *d_out, size_t n, uint64_t seed,
                              fg_stream_t stream);

/* Streaming device copy of `bytes` (a multiple of 16; both pointers 16-byte
 * aligned) with the code object's copy kernel: the HBM yardstick reported
 * beside the FFT. */
FG_API int fg_stream_copy(fg_device_t dev, const void *d_in, void *d_out, size_t bytes,
                   fg_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* FERRUM_GPU_H */
