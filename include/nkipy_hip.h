/*
 * nkipy_hip.h -- C ABI of libnkipy_hip.so, the native runtime under the
 * NKIPy MI355X backend.
 *
 * This library replaces the Spike/libnrt layer of the reference
 * (spike/src/*.cpp, bound through nanobind in spike/src/python_bindings.cpp)
 * with a thin layer over the HIP runtime and module APIs.  It is loaded
 * from Python with ctypes; no torch or Python types appear in the ABI.
 *
 * Conventions
 *   - Every function returns an int status: NKH_OK (0) on success.
 *   - On failure nkh_last_error() returns a thread-local message.
 *   - One device and one non-blocking stream (default priority) per process,
 *     selected by nkh_init().  Launches are asynchronous on that stream;
 *     nkh_sync() waits for it.
 *   - Device pointers returned by nkh_malloc() are owned by the caller until
 *     nkh_free().  The runtime keeps a registry of live allocations, so a
 *     copy that runs past the end of an allocation, or touches a freed one,
 *     is rejected with NKH_ERR_BOUNDS / NKH_ERR_FREED instead of faulting.
 *   - nkh_shutdown() frees every allocation and module still registered.
 */
#ifndef NKIPY_HIP_H
#define NKIPY_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  NKH_ERR_HIP carries the hipError_t name in the message
 * (the analogue of NrtError, spike/src/include/error.h:23-44); the other
 * codes are runtime-level errors (the analogue of SpikeError, error.h:17-21). */
enum {
  NKH_OK = 0,
  NKH_ERR_HIP = 1,         /* a HIP call failed */
  NKH_ERR_INVALID = 2,     /* bad argument (null pointer, zero size, ...) */
  NKH_ERR_NOT_INIT = 3,    /* nkh_init() has not run, or nkh_shutdown() ran */
  NKH_ERR_BOUNDS = 4,      /* copy or memset past the end of an allocation */
  NKH_ERR_FREED = 5,       /* pointer is not (or no longer) a live allocation */
  NKH_ERR_ALREADY_INIT = 6 /* nkh_init() called twice without shutdown */
};

/* Last error message of the calling thread ("" if none).
 * Replaces the exception text of SpikeError/NrtError. */
const char *nkh_last_error(void);

/* Runtime lifetime.  Replaces NrtRuntime (spike/src/nrt_wrapper.cpp:47-75)
 * and the Spike constructor/close (spike/src/spike.cpp:6-41): a second init
 * without shutdown fails like a second Spike instance (spike.cpp:11-16). */
int nkh_init(int device);
int nkh_shutdown(void);
int nkh_is_initialized(int *flag);

/* Device queries.  nkh_device_count replaces
 * Spike::get_visible_neuron_core_count (spike/src/spike.cpp:27-29).
 * nkh_device_info reports what the roofline derivation needs:
 * compute-unit count, peak shader clock (kHz), memory clock (kHz),
 * memory bus width (bits), L2 size (bytes) and the gfx arch name. */
int nkh_device_count(int *count);
int nkh_device_info(int *cu_count, int *clock_khz, int *mem_clock_khz,
                    int *mem_bus_bits, int *l2_bytes, char *arch_name,
                    size_t arch_name_len);

/* Device memory.  Replaces NrtTensor allocate/free/read/write
 * (spike/src/tensor.cpp:9-115; Spike::allocate_tensor,
 * tensor_write_from_pybuffer, tensor_read_to_pybuffer in
 * spike/src/spike.cpp:43-86).  Copies are synchronous with respect to the
 * runtime stream (they wait for queued launches), like nrt_tensor_read/
 * write.  `dst`/`src` device pointers may point inside an allocation; the
 * whole range must stay inside it. */
int nkh_malloc(size_t bytes, void **ptr);
int nkh_free(void *ptr);
int nkh_alloc_size(const void *ptr, size_t *bytes);
int nkh_memcpy_h2d(void *dst, const void *src, size_t bytes);
int nkh_memcpy_d2h(void *dst, const void *src, size_t bytes);
int nkh_memcpy_d2d(void *dst, const void *src, size_t bytes);
int nkh_memset(void *ptr, int value, size_t bytes);

/* Code objects.  Replaces NrtModel load/unload of a NEFF
 * (spike/src/model.cpp:10-88): a module is a gfx950 code object (.hsaco)
 * built ahead of time by hipcc; functions are looked up by symbol. */
int nkh_module_load(const char *hsaco_path, void **module);
int nkh_module_unload(void *module);
int nkh_get_function(void *module, const char *symbol, void **function);

/* Kernel launch on the runtime stream.  `kernarg` is the packed argument
 * block of the kernel (HIP_LAUNCH_PARAM_BUFFER_POINTER).  Replaces
 * NrtModel::execute / nrt_execute (spike/src/model.cpp:90-110), except that
 * it is asynchronous: nkh_sync() gives nrt_execute's completion point. */
int nkh_launch(void *function, unsigned gx, unsigned gy, unsigned gz,
               unsigned bx, unsigned by, unsigned bz, unsigned shared_bytes,
               const void *kernarg, size_t kernarg_bytes);
int nkh_sync(void);

/* Device timing of one kernel: `warmup` untimed launches, then `iters`
 * launches bracketed by HIP events on the runtime stream; *ms_out is the
 * mean time per launch.  Replaces SpikeModel.benchmark(mode="device")
 * (spike/src/spike/spike_model.py:270-330), which reads device timestamps
 * from the NRT system trace (spike/src/sys_trace.cpp:5-103). */
int nkh_time_launch(void *function, unsigned gx, unsigned gy, unsigned gz,
                    unsigned bx, unsigned by, unsigned bz,
                    unsigned shared_bytes, const void *kernarg,
                    size_t kernarg_bytes, int warmup, int iters,
                    float *ms_out);

/* Events on the runtime stream, for timing a sequence of launches.
 * Same role as the sys-trace session above. */
int nkh_event_create(void **event);
int nkh_event_destroy(void *event);
int nkh_event_record(void *event);
int nkh_event_elapsed_ms(void *start, void *stop, float *ms_out);

/* Named profiler ranges around a stretch of host calls (roctx ranges,
 * shown by `rocprofv3 --marker-trace`).  They stand where the reference
 * brackets one execution with nrt_profile_start / nrt_profile_stop
 * (spike/src/model.cpp:97-103).  The roctx library is opened on first use;
 * where it is absent both calls succeed and record nothing, and *available
 * (if not null) reports 0.  Ranges nest per thread; a pop without a push
 * returns NKH_ERR_INVALID. */
int nkh_profile_range_push(const char *name, int *available);
int nkh_profile_range_pop(void);

/* Batched launch: run `count` launches back to back on the runtime stream
 * with one host call.  Launch i uses functions[i], grids[3i..3i+2],
 * blocks[3i..3i+2], shared[i] and the kernarg block at
 * kernargs + kernarg_offsets[i] of kernarg_sizes[i] bytes.  This is the
 * prebuilt-argument replay path for a compiled kernel plan (the per-call
 * work of SpikeModel.__call__, spike/src/spike/spike_model.py:228-268,
 * reduced to one native call). */
int nkh_launch_batch(int count, void *const *functions,
                     const unsigned *grids, const unsigned *blocks,
                     const unsigned *shared, const uint8_t *kernargs,
                     const size_t *kernarg_offsets,
                     const size_t *kernarg_sizes);

/* Graph replay of a batch: the launches of nkh_launch_batch (same arrays,
 * count >= 1) are captured once from the runtime stream into a HIP graph,
 * which nkh_graph_launch replays on that stream with one host call and no
 * per-launch argument handling: the argument blocks are copied at capture,
 * so the device addresses in them are fixed for the graph's lifetime.  The
 * reference replays a loaded model through nrt_execute per call
 * (spike/src/model.cpp:90-110); this is that replay for serving loops whose
 * host dispatch of many small launches would otherwise show.  Graphs are
 * released by nkh_graph_destroy (which drains the stream first) or at
 * nkh_shutdown; a handle not created by this runtime, or already destroyed,
 * is NKH_ERR_INVALID. */
int nkh_graph_create(int count, void *const *functions,
                     const unsigned *grids, const unsigned *blocks,
                     const unsigned *shared, const uint8_t *kernargs,
                     const size_t *kernarg_offsets,
                     const size_t *kernarg_sizes, void **graph);
int nkh_graph_launch(void *graph);
int nkh_graph_destroy(void *graph);

/* Chunked causal linear attention, phi = elu + 1, chunk 64, d = d_v = 128:
 * o[s, t, :] = sum_{u<=t} (phi(q_t).phi(k_u)) v_u / sum_{u<=t} phi(q_t).phi(k_u)
 * over `bh` sequences of `t` tokens; q, k, v, o are (bh, t, 128) bf16,
 * row-major, 16-byte aligned.  Asynchronous on the runtime stream.
 *
 * The reference has no kernel for this (its nearest analogue is the
 * recurrent DeltaNet kernel, examples/linear_attention/deltanet.py:74-128,
 * run through nrt_execute, spike/src/model.cpp:90-110); this is the entry
 * point a ctypes caller binds instead of tracing the NumPy kernel.
 *
 * With few sequences the scan is cut into segments whose prefix states go
 * through `workspace` (device memory of at least the size
 * nkh_linear_attention_workspace_size reports; 0 bytes means none is
 * needed and `workspace` may be null).  The workspace is fully written
 * before it is read: it needs no clearing. */
int nkh_linear_attention_workspace_size(int64_t bh, int64_t t, size_t *bytes);
int nkh_linear_attention(const void *q, const void *k, const void *v, void *o,
                         int64_t bh, int64_t t, void *workspace,
                         size_t workspace_size);

/* nkh_linear_attention without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The partial prefix states go to a scratch array of
 * NKH_NOALLOC_SCRATCH_BYTES that the library keeps on each device it was
 * initialized on until the process ends; shapes whose workspace exceeds it
 * are rejected with NKH_ERR_INVALID (use nkh_linear_attention then).  The
 * call allocates and frees nothing.  Every call on a GPU shares that GPU's
 * array: calls queued on the runtime stream run one after another, but
 * calls that overlap on one GPU (another stream or process driving the
 * same library state) race.  The array needs no clearing: each call writes
 * every partial state before reading it. */
#define NKH_NOALLOC_SCRATCH_BYTES (16u << 20)
int nkh_linear_attention_noalloc(const void *q, const void *k, const void *v,
                                 void *o, int64_t bh, int64_t t);

#ifdef __cplusplus
}
#endif

#endif /* NKIPY_HIP_H */
