/*
 * palladium_hip: the C ABI between palladium_amd's Python host layer (or a
 * jax.ffi handler) and the HIP runtime on MI355X (gfx950).
 *
 * Everything crossing this boundary is a plain pointer, size or integer.
 * Every function returns PH_OK (0) or an error code and, where it takes a
 * `char **err`, stores a heap message there that the caller releases with
 * ph_free_error().
 *
 * Each entry point names the reference interface it replaces
 * (paths relative to nicholasjng/palladium).
 */
#ifndef PALLADIUM_HIP_H
#define PALLADIUM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  PH_OK = 0,
  PH_ERR_INVALID_ARGUMENT = 1,
  PH_ERR_COMPILE = 2,
  PH_ERR_RUNTIME = 3,
};

/* Math modes, same ordinals as the reference's MRMathMode
 * (src/palladium/ffi.py:38): SAFE = IEEE order, no contraction;
 * RELAXED = FMA contraction; FAST = contraction, reassociation and
 * approximate transcendentals/division (infinities and NaNs still honoured).
 * PH_MATH_REPRODUCIBLE (no counterpart in the reference; the reference's
 * handler rejects 3 with InvalidArgument): FAST's algebra with fused
 * multiply-adds at the sites the emitter writes out, division as a times
 * the correctly rounded 1/b, and deterministic pow/log2/exp2, so a host
 * restates the results bit for bit (compiled with -ffp-contract=off). */
enum { PH_MATH_SAFE = 0, PH_MATH_RELAXED = 1, PH_MATH_FAST = 2, PH_MATH_REPRODUCIBLE = 3 };

typedef struct ph_kernel ph_kernel;

/* Library version string, e.g. "0.1.0". */
const char *ph_version(void);

/* Releases a message returned through an `err` out-parameter.
 * Replaces mr_free_error_message (native/ffi/palladium_ffi.cpp:60-61). */
void ph_free_error(char *err);

/* Compiles HIP source with hiprtc for `arch` (NULL = "gfx950") and returns
 * the code object (release with ph_free_code_object). Needs no GPU.
 * Replaces mr_compile_library (native/ffi/palladium_ffi.cpp:57-58). */
int ph_compile_code_object(const char *src, size_t src_len, const char *name,
                           int math_mode, const char *arch, void **code,
                           size_t *code_size, char **err);
void ph_free_code_object(void *code);

/* The math-mode-specific hiprtc options (static storage). Every compile
 * also passes --offload-arch, -O3, -std=c++17, -fwrapv, -fno-slp-vectorize,
 * -DPH_MATH_MODE=<mode> and disables the packed FP32 target feature. */
const char *ph_compile_options(int math_mode);

/* Compile (outside the cache lock), load on the current device and look up
 * `name`; cached for the process lifetime by (source, name, math mode,
 * device). Concurrent first calls may compile twice; the loser is unloaded.
 * Replaces KernelCache::get_or_compile (native/ffi/palladium_ffi.cpp:25-91)
 * plus mr_get_pipeline. */
int ph_get_kernel(const char *src, size_t src_len, const char *name,
                  int math_mode, ph_kernel **out, char **err);

/* Load a code object made by ph_compile_code_object (possibly in another
 * process) on the current device and look up `name`. The kernel lives for
 * the rest of the process; callers cache it. No reference counterpart:
 * metal-runtime compiles and loads in one step. It lets a host compile in a
 * helper process, where a compiler crash cannot end the caller. */
int ph_load_code_object(const void *code, size_t code_size, const char *name,
                        ph_kernel **out, char **err);

/* Number of distinct kernels in the cache (for tests). */
size_t ph_kernel_cache_size(void);

/* Launch on `stream` (NULL = default stream), asynchronously. `params` is
 * the hipModuleLaunchKernel argument array (one pointer to each argument
 * value). Replaces the dispatch half of mr_dispatch
 * (native/ffi/palladium_ffi.cpp:150-165). */
int ph_launch(ph_kernel *k, unsigned int grid_x, unsigned int grid_y,
              unsigned int grid_z, unsigned int block_x, unsigned int block_y,
              unsigned int block_z, unsigned int shared_bytes, void *stream,
              void **params, char **err);

/* Launch a kernel whose arguments are exactly `n_ptrs` device pointers
 * (the signature emit_hip produces), over a 1-D grid. */
int ph_launch_ptrs(ph_kernel *k, unsigned int blocks, unsigned int block,
                   void *stream, void *const *ptrs, size_t n_ptrs, char **err);

/* One synchronous dispatch of emitted source over host buffers: compile or
 * hit the cache, stage inputs host->device, launch
 * ceil(prod(grid) * lanes / block) workgroups of `block` threads (0 = 256),
 * copy outputs device->host, wait. Attribute-for-attribute the reference's
 * XLA FFI handler on the "cpu" platform (native/ffi/palladium_ffi.cpp:
 * 110-209): source, function name, grid, block (threadgroup), math mode,
 * then inputs, then outputs; plus `lanes`, the threads per program instance
 * (1, or the block rows a lane-parallel kernel spreads across lanes), which
 * Metal's one-thread-per-instance model has no use for. */
int ph_dispatch(const char *src, size_t src_len, const char *name,
                int64_t grid_x, int64_t grid_y, int64_t grid_z,
                int64_t block_x, int64_t lanes, int64_t math_mode,
                const void *const *inputs, const size_t *input_bytes,
                size_t n_inputs, void *const *outputs,
                const size_t *output_bytes, size_t n_outputs, char **err);

/* The same dispatch over device buffers on the caller's stream: no
 * staging, no allocation beyond the compile cache, no wait (the launch is
 * ordered on `stream`; NULL = default stream). The body an XLA FFI handler
 * on the "ROCM" platform needs (device buffers + the XLA stream), which the
 * reference's Metal-only native/ffi/palladium_ffi.cpp:110-193 has no
 * counterpart for. */
int ph_dispatch_device(const char *src, size_t src_len, const char *name,
                       int64_t grid_x, int64_t grid_y, int64_t grid_z,
                       int64_t block_x, int64_t lanes, int64_t math_mode,
                       void *stream, const void *const *inputs,
                       size_t n_inputs, void *const *outputs,
                       size_t n_outputs, char **err);

/* Staging objects ph_dispatch has created so far (a stream, device buffers
 * and a pinned bounce buffer each). A thread holds one per device while it
 * lives and returns it to a pool at exit for the next thread, so the count
 * grows only with the threads dispatching at once. For tests. */
size_t ph_dispatch_staging_count(void);

/* Size of the fixed device scratch area of ph_dispatch_noalloc, per GPU. */
#define PH_NOALLOC_SCRATCH_BYTES (64u << 20)
size_t ph_noalloc_scratch_bytes(void);

/* No counterpart in the reference. ph_dispatch for callers that cannot
 * allocate: serving loops and harnesses that forbid hipMalloc/hipFree.
 * It calls no hipMalloc, hipFree, hipHostMalloc, stream creation, compiler
 * or module loader, and no allocating library routine:
 *  - `k` comes from an earlier ph_get_kernel or ph_load_code_object on the
 *    current device (emitted source carries its math mode);
 *  - operands are staged in one fixed device array of
 *    PH_NOALLOC_SCRATCH_BYTES (64 MiB) per GPU, reserved on every GPU where
 *    this library's code object loads (whether or not this entry point is
 *    ever called) and held until the process ends, each operand at a 256-byte boundary in argument order; operands
 *    that do not fit are rejected with PH_ERR_INVALID_ARGUMENT before
 *    anything is queued;
 *  - output slots are cleared to zero before the launch;
 *  - the work is ordered on `stream` (NULL = default stream) and the call
 *    returns once the outputs are in the caller's host buffers.
 * Launch geometry and operand order are ph_dispatch's. Every call on one
 * GPU shares that GPU's array, so calls on one GPU are serialised by a
 * per-GPU lock held from the first copy in to the synchronisation after the
 * last copy out: threads that call at once wait for each other (the array
 * belongs to this process; other processes have their own). */
int ph_dispatch_noalloc(ph_kernel *k, int64_t grid_x, int64_t grid_y, int64_t grid_z,
                        int64_t block_x, int64_t lanes, void *stream,
                        const void *const *inputs, const size_t *input_bytes,
                        size_t n_inputs, void *const *outputs,
                        const size_t *output_bytes, size_t n_outputs, char **err);

/* Device memory, streams, events and graphs: the role metal-runtime's
 * Buffer/Batch/gpu_time play for the reference
 * (src/palladium/dispatch.py:18,183-225). Streams are created at the
 * default priority. */
int ph_device_count(int *count);
int ph_device_name(char *buf, size_t len);
int ph_malloc(size_t bytes, void **ptr, char **err);
int ph_free(void *ptr);
/* Pinned (page-locked) host memory, the staging a device->host copy can run
 * into asynchronously (metal-runtime needs none: unified memory). */
int ph_host_alloc(size_t bytes, void **ptr, char **err);
int ph_host_free(void *ptr);
int ph_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream, char **err);
int ph_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream, char **err);
/* Device -> host copy ordered on `stream`, returning once `dst` holds the
 * data (the readback half of a dispatch; small copies bounce through a
 * per-thread pinned buffer). */
int ph_memcpy_d2h_wait(void *dst, const void *src, size_t bytes, void *stream, char **err);
int ph_memcpy_d2d(void *dst, const void *src, size_t bytes, void *stream, char **err);
int ph_stream_create(void **stream, char **err);
int ph_stream_destroy(void *stream);
int ph_stream_synchronize(void *stream, char **err);
int ph_event_create(void **event, char **err);
int ph_event_destroy(void *event);
int ph_event_record(void *event, void *stream, char **err);
int ph_event_synchronize(void *event, char **err);
int ph_event_query(void *event); /* 1 = complete, 0 = pending, <0 error */
int ph_event_elapsed_ms(void *start, void *stop, float *ms, char **err);
int ph_device_synchronize(char **err);

/* Stream capture into a HIP graph and replay: the multi-launch batch of
 * the reference's Gray-Scott driver (examples/04_reaction_diffusion.py:
 * 100-107) as one graph launch. */
int ph_stream_begin_capture(void *stream, char **err);
int ph_stream_end_capture(void *stream, void **graph_exec, char **err);
int ph_graph_launch(void *graph_exec, void *stream, char **err);
int ph_graph_destroy(void *graph_exec);

#ifdef __cplusplus
}
#endif

#endif /* PALLADIUM_HIP_H */
