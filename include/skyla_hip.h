/*
 * skyla_hip.h -- C-ABI of the MI355X (gfx950) backend for Skyla's quantized weight path.
 *
 * This is the surface skyla-engine reaches through `crate::gpu` (the module that
 * skyla-engine/src/backend.rs:1-19 swaps between skyla_vk and skyla_metal).  Each entry
 * point names the reference method it replaces.  Plain pointers and sizes only; no HIP
 * or torch types cross this boundary.
 *
 * Conventions
 *   - Every function returning int returns SKYLA_HIP_OK (0) or a negative error code;
 *     skyla_hip_last_error() then holds a message for the calling thread (the anyhow
 *     context the Rust backends attach).  Nothing aborts across the boundary.
 *   - Handles are opaque.  As with the Rust lifetimes in skyla-engine/src/engine.rs:12-22,
 *     buffers must outlive the pipelines bound to them and the recordings that use
 *     those pipelines, and everything must be freed before its context.
 *   - One context owns one HIP stream.  Calls on one context must be serialised by the
 *     caller (the reference types are !Sync: skyla-vk/src/record.rs:21).
 *   - Push words are u32 in the order of the reference's push layouts; floats are
 *     passed as their bit patterns (f32::to_bits).  Offsets inside push words are
 *     element indices in the unit of the binding they address (uvec4 = 16 B for
 *     weight regions, f16 for scale arrays, f32/u32 for the arena).
 */
#ifndef SKYLA_HIP_H
#define SKYLA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SKYLA_HIP_OK 0
#define SKYLA_HIP_E_ARG (-1)       /* bad argument (null handle, size, index) */
#define SKYLA_HIP_E_DEVICE (-2)    /* no device, or a HIP runtime call failed */
#define SKYLA_HIP_E_NO_KERNEL (-3) /* no kernel for this (name, spec) */
#define SKYLA_HIP_E_OOM (-4)       /* allocation failed or above max_buffer */
#define SKYLA_HIP_E_STATE (-5)     /* call not valid in this state */

typedef struct skyla_hip_context skyla_hip_context;
typedef struct skyla_hip_buffer skyla_hip_buffer;
typedef struct skyla_hip_pipeline skyla_hip_pipeline;
typedef struct skyla_hip_recorder skyla_hip_recorder;
typedef struct skyla_hip_recording skyla_hip_recording;

/* Message of the last failed call on this thread ("" if none). */
const char *skyla_hip_last_error(void);

/* ---- Context (skyla-vk/src/context.rs:85 Context::new; engine.rs:48) ---- */

/* Opens device `device` (SKYLA_DEVICE in skyla-vk/src/context.rs:50-55 picks the index
 * the same way), creates its stream and loads the embedded gfx950 code object. */
int skyla_hip_context_new(int device, skyla_hip_context **out);
void skyla_hip_context_free(skyla_hip_context *ctx);
/* Context::subgroup_size (kernels.rs:93): 64 on gfx950. */
uint32_t skyla_hip_subgroup_size(const skyla_hip_context *ctx);
/* Context::max_buffer (weights.rs:62, arena.rs:149): 4 GiB, so u32 element offsets
 * of every binding type stay in range. */
uint64_t skyla_hip_max_buffer(const skyla_hip_context *ctx);
/* Context::device_name (skyla-vk/src/context.rs:169; engine.rs:71).  Writes a NUL-terminated name into out[cap]. */
int skyla_hip_device_name(const skyla_hip_context *ctx, char *out, size_t cap);

/* ---- Buffer (skyla-vk/src/buffer.rs:6-35 Buffer; 49-62 max_buffer, alloc_host) ---- */

/* Context::alloc_host: `size` bytes of HBM plus a host mirror the engine fills through
 * skyla_hip_buffer_host (Buffer::as_mut_slice / as_f32_mut / as_u32_mut).  HBM starts
 * zeroed.  Fails above max_buffer. */
int skyla_hip_alloc(skyla_hip_context *ctx, uint64_t size, skyla_hip_buffer **out);
void skyla_hip_buffer_free(skyla_hip_buffer *buf);
/* Buffer::size (engine.rs:75). */
uint64_t skyla_hip_buffer_size(const skyla_hip_buffer *buf);
/* Host mirror of the buffer (Buffer::as_mut_slice).  The reference's buffers are
 * host-coherent; on a discrete MI355X the mirror is synchronised explicitly with the
 * two calls below, at the four places the engine touches buffer memory from the host
 * (after Planner::fill, after Engine::load, before logits and taps reads). */
void *skyla_hip_buffer_host(skyla_hip_buffer *buf);
/* Copies host mirror [off, off+len) to HBM, and back. Synchronous on the context stream. */
int skyla_hip_buffer_upload(skyla_hip_buffer *buf, uint64_t off, uint64_t len);
int skyla_hip_buffer_download(skyla_hip_buffer *buf, uint64_t off, uint64_t len);
/* Device address of the buffer, for callers that fill HBM themselves. */
void *skyla_hip_buffer_device(skyla_hip_buffer *buf);
/* Device-to-device copy between buffers, on the context stream, synchronous. */
int skyla_hip_buffer_copy(skyla_hip_buffer *dst, uint64_t dst_off, const skyla_hip_buffer *src,
                          uint64_t src_off, uint64_t len);

/* ---- Pipeline (skyla-vk/src/pipeline.rs:16-124; kernels.rs:60, 118-119) ---- */

/* Context::create_pipeline_sets(shader, n_buffers, push_size, spec, n_sets).
 * `name` is the reference shader name (matvec_q4k, matvec_q6k, matvec_q8_0, matmul,
 * moe_logits, moe_route, moe_sort, moe_combine, silu_mul, to_half, bandwidth).  The
 * kernel is the gfx950 instantiation for `spec`; an unknown (name, spec) fails with
 * SKYLA_HIP_E_NO_KERNEL, as a shader that does not compile fails pipeline creation.
 * n_buffers and push_size must match the kernel's bindings and push struct.
 * A matvec pipeline (dense rows, or Q4_K expert rows) may launch another compiled variant
 * of the same kernel (same bindings and push words, different rows per workgroup) chosen
 * by the launch's total rows, with grid.x recomputed from each dispatch's n_out (grid.y,
 * the expert slots, is kept); every row is
 * still computed once, and results differ from the requested variant only by f32
 * summation order.  Environment SKYLA_HIP_RETILE=0 (read here) keeps the requested one. */
int skyla_hip_pipeline_new(skyla_hip_context *ctx, const char *name, uint32_t n_buffers,
                           uint32_t push_size, const uint32_t *spec, uint32_t n_spec,
                           uint32_t n_sets, skyla_hip_pipeline **out);
void skyla_hip_pipeline_free(skyla_hip_pipeline *p);
/* Pipeline::bind_set_buffers(set, buffers) (pipeline.rs:104-124); bind_buffers (:100) is set 0. */
int skyla_hip_pipeline_bind(skyla_hip_pipeline *p, uint32_t set, skyla_hip_buffer *const *bufs,
                            uint32_t n);
/* Threads per workgroup for this pipeline (the per-kernel shape table of
 * skyla-metal/src/pipeline.rs:14-24, made explicit). */
int skyla_hip_pipeline_threads(const skyla_hip_pipeline *p, uint32_t out[3]);

/* ---- Record / replay (skyla-vk/src/record.rs:8-57 Recording, Recorder; 83-148 record, replay, marks) ---- */

/* Context::record(profile, f): begin, issue Recorder calls, end. */
int skyla_hip_record_begin(skyla_hip_context *ctx, int profile, skyla_hip_recorder **out);
/* Recorder::dispatch_set(p, set, groups, push) / Recorder::dispatch (set 0). */
int skyla_hip_record_dispatch(skyla_hip_recorder *r, const skyla_hip_pipeline *p, uint32_t set,
                              const uint32_t groups[3], const uint32_t *push, uint32_t n_push);
/* Recorder::barrier: every later dispatch sees the writes of every earlier one.
 * Dispatches between two barriers are independent of each other. */
int skyla_hip_record_barrier(skyla_hip_recorder *r);
/* Recorder::host_barrier: results are visible to the host after replay returns. */
int skyla_hip_record_host_barrier(skyla_hip_recorder *r);
/* Recorder::mark(label): a timestamp after all work recorded so far (profiled only). */
int skyla_hip_record_mark(skyla_hip_recorder *r, const char *label);
/* Ends recording; the recorder is consumed whatever the result. */
int skyla_hip_record_end(skyla_hip_recorder *r, skyla_hip_recording **out);
void skyla_hip_recording_free(skyla_hip_recording *rec);
/* Number of dispatches in a recording. */
uint32_t skyla_hip_recording_len(const skyla_hip_recording *rec);
/* Number of kernel launches a replay makes (no counterpart in the reference, whose
 * Vulkan command buffer issues one dispatch per Recorder::dispatch).  Consecutive
 * dispatches of one matvec pipeline with no barrier between them, which the engine's
 * contract makes independent, are fused into one launch over their combined rows
 * (at most 4; environment SKYLA_HIP_FUSE=0 turns this off).  Profilers see launches. */
uint32_t skyla_hip_recording_launches(const skyla_hip_recording *rec);

/* Context::replay: run the recording (as one HIP graph) and wait for it. */
int skyla_hip_replay(skyla_hip_context *ctx, const skyla_hip_recording *rec);
/* Replay and report the device time between its first and last work, in ns, measured
 * with HIP events on the context stream. */
int skyla_hip_replay_timed(skyla_hip_context *ctx, const skyla_hip_recording *rec,
                           double *ns);
/* Context::marks (record.rs:137-148): for a profiled recording, after a replay.
 * Fills up to `cap` entries of label pointers (valid while the recording lives) and
 * ns deltas; *count receives the number of marks. */
int skyla_hip_marks(skyla_hip_context *ctx, const skyla_hip_recording *rec,
                    const char **labels, double *ns, uint32_t cap, uint32_t *count);

/* Context::time_dispatch(pipeline, groups, push, reps) (skyla-vk/src/submit.rs:31-76):
 * `reps` back-to-back dispatches of set 0, ns per dispatch into ns_out[reps]. */
int skyla_hip_time_dispatch(skyla_hip_context *ctx, const skyla_hip_pipeline *p,
                            const uint32_t groups[3], const uint32_t *push, uint32_t n_push,
                            uint32_t reps, double *ns_out);

/* No counterpart in the reference.  For callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): one
 * dispatch of set 0 of `p`, as skyla_hip_time_dispatch makes with reps = 1, untimed and
 * synchronous, with no hipMalloc, hipFree or other allocating call.  The one kernel family
 * that needs a workspace, the K split of a dense K-quant matmul, takes its partial tiles
 * and counters from a static device array of this context's matmul code object (256 f32
 * tiles of 128 x 128 and 1024 counters: 16 MiB + 4 KiB) instead of a workspace of its
 * own; a launch needing more fails with SKYLA_HIP_E_OOM.  Every call on one context shares
 * that array: calls that overlap (several host threads, or work still queued on the
 * context stream by another caller) race. */
int skyla_hip_dispatch_noalloc(skyla_hip_context *ctx, const skyla_hip_pipeline *p,
                               const uint32_t groups[3], const uint32_t *push, uint32_t n_push);

#ifdef __cplusplus
}
#endif
#endif
