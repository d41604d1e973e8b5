/*
 * axon_hip.h — C ABI of the gfx950 kernel library (libaxon_hip.so).
 *
 * The reference (akothen/enzyme, package `axon`) has no native library: its
 * boundary between host and device is a generated kernel module plus two
 * worker calls. Each entry point below replaces one piece of that boundary:
 *
 *   axon_kernel_variants / axon_variant_describe
 *       the set of per-variant modules the NKI emitter writes
 *       (src/axon/codegen/assemble.py:824-860, discovered by
 *       src/axon/cli.py:307-354);
 *   axon_variant_manifest
 *       the literal `__axon_tile_constraints__` manifest each module carries
 *       (src/axon/codegen/assemble.py:495-595, read by
 *       src/axon/candidate_filter.py:56-87);
 *   axon_variant_check
 *       the compile worker's legality verdict for one TILES_IN_BLOCK_* tuple,
 *       where an AssertionError with no artefact means an illegal tile
 *       configuration (src/axon/bench_runner.py:226-272);
 *   axon_variant_workspace / axon_variant_launch
 *       running the compiled kernel on device buffers with its tile values
 *       baked in (src/axon/bench_runner.py:144-223: inputs by name in
 *       `input_specs` order, outputs in `out_0..out_k` order);
 *   axon_copy / axon_copy_shape
 *       no counterpart in the reference: a plain device copy of known size
 *       used to calibrate HBM traffic counters and to measure the fastest
 *       copy of a given size;
 *   axon_scan_poll_bound
 *       no counterpart in the reference (whose scan is a sequential carry,
 *       winners/cumsum_llama3_vocab.py:57-75): sets how long the single-pass
 *       cumsum variant waits for an earlier chunk's published total before
 *       recomputing it from the input.
 *
 * Conventions: every call returns AXON_OK (0) or an AXON_E* code, and never
 * throws; `axon_last_error` gives the calling thread's last message. Device
 * buffers belong to the caller (contiguous, row-major, in the spec's declared
 * layout); a workspace, when one is needed, is caller-owned too. Launches are
 * asynchronous on `stream`. The registry is immutable, so every entry point
 * is reentrant. The check/manifest/describe calls run on the host only and
 * never initialise the HIP runtime.
 */
#ifndef AXON_HIP_H
#define AXON_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AXON_ABI_VERSION 1

enum axon_status {
  AXON_OK = 0,
  AXON_EINVAL = 1,      /* illegal tile tuple or shape for this variant */
  AXON_ENOKERNEL = 2,   /* unknown kernel name or hw_variant index */
  AXON_EDTYPE = 3,      /* unsupported input dtype combination */
  AXON_EARG = 4,        /* wrong argument count / null pointer / misalignment */
  AXON_EWORKSPACE = 5,  /* workspace missing or too small */
  AXON_EHIP = 6,        /* a HIP runtime call failed (see axon_last_error) */
  AXON_EBUFFER = 7      /* caller buffer too small for the text result */
};

enum axon_dtype {
  AXON_BF16 = 0,
  AXON_F16 = 1,
  AXON_F32 = 2
};

/* hipStream_t without pulling in the HIP headers. */
typedef struct ihipStream_t* axon_stream_t;

int axon_abi_version(void);
const char* axon_last_error(void);

/* Number of kernel families in the registry and the spec name of each. */
int axon_kernel_count(void);
const char* axon_kernel_name(int index);

/* Number of hw variants for a spec name (0 when the name is unknown). */
int axon_kernel_variants(const char* kernel);

/* JSON object describing variant `hw_variant`: tile argument names in order,
 * input/output counts, and a one-line summary of its schedule. */
int axon_variant_describe(const char* kernel, int hw_variant, char* buf,
                          size_t buf_len);

/* The tile manifest for one binding of the spec's dim_vars, as JSON:
 * {"version": 1, "constraints": [{"tile_arg": ..., "extent": ...,
 *  "tile_size": ..., "require_divisible": ...}, ...]}. `dtype` is the
 * element type of input 0 (it sets the 16-byte vector width). */
int axon_variant_manifest(const char* kernel, int hw_variant,
                          const int64_t* dims, int n_dims, int dtype,
                          char* buf, size_t buf_len);

/* Shapes and element types of a spec's outputs (independent of the hw
 * variant): writes ranks[i], out_dtypes[i] and shapes[i*max_rank + k] for
 * each output i (out_0..out_k order) and returns the output count, or a
 * negated AXON_E* code. Replaces reading the compiled kernel's output tensor
 * table (src/axon/bench_runner.py:196-201). */
int axon_variant_outputs(const char* kernel, const int64_t* dims, int n_dims,
                         const int32_t* dtypes, int n_dtypes, int max_rank,
                         int64_t* shapes, int32_t* ranks, int32_t* out_dtypes,
                         int cap);

/* AXON_OK when the tile tuple is instantiated and legal for these dims and
 * input dtypes (one code per input, in input_specs order); AXON_EINVAL
 * otherwise, with the reason in axon_last_error(). */
int axon_variant_check(const char* kernel, int hw_variant,
                       const int32_t* tiles, int n_tiles,
                       const int64_t* dims, int n_dims,
                       const int32_t* dtypes, int n_dtypes);

/* Bytes of device workspace one launch needs (0 for most variants). A
 * workspace must be zero-filled before its first launch; every launch leaves
 * it ready for the next one (the single-pass cumsum variant keeps a count of
 * recomputed chunk totals in its first word). Launches that overlap on one
 * workspace race. */
size_t axon_variant_workspace(const char* kernel, int hw_variant,
                              const int32_t* tiles, int n_tiles,
                              const int64_t* dims, int n_dims,
                              const int32_t* dtypes, int n_dtypes);

/* Enqueue one launch. Performs the same checks as axon_variant_check plus
 * pointer alignment and workspace size, and enqueues nothing on failure.
 * When every output has zero elements the launch is a no-op that returns
 * AXON_OK without looking at the pointers (empty buffers may be null). */
int axon_variant_launch(const char* kernel, int hw_variant,
                        const int32_t* tiles, int n_tiles,
                        const int64_t* dims, int n_dims,
                        const int32_t* dtypes, int n_dtypes,
                        const void* const* inputs, int n_in,
                        void* const* outputs, int n_out,
                        void* workspace, size_t workspace_bytes,
                        axon_stream_t stream);

/* As axon_variant_launch, but allocates nothing and takes no workspace. No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). The kernels' workspace is a static device
 * array of 32 MiB per GPU, held until the process ends; a launch that needs
 * more returns AXON_EWORKSPACE (sizes in axon_last_error()) and enqueues
 * nothing. The first call on a device looks the array's address up
 * (hipGetSymbolAddress); no call allocates or frees memory. Every call on a
 * GPU shares that GPU's array and it keeps the last call's contents: the part
 * a kernel needs at zero is cleared by a small fill kernel on `stream` before
 * the launch. Calls whose execution can overlap on one GPU (unordered streams,
 * or several threads) race. */
int axon_variant_launch_noalloc(const char* kernel, int hw_variant,
                                const int32_t* tiles, int n_tiles,
                                const int64_t* dims, int n_dims,
                                const int32_t* dtypes, int n_dtypes,
                                const void* const* inputs, int n_in,
                                void* const* outputs, int n_out,
                                axon_stream_t stream);

/* Copy `bytes` (a multiple of 16, both pointers 16-byte aligned) on `stream`
 * with a plain vector-copy kernel: the known-size reference for traffic
 * counters. Same as axon_copy_shape with shape 0. */
int axon_copy(const void* src, void* dst, size_t bytes, axon_stream_t stream);

/* The same copy in one of four launch shapes, to measure the fastest plain
 * copy of a given size (the HBM ceiling a streaming kernel of that size can
 * reach): 0 = one 16-byte vector per thread per step, grid-stride over at
 * most 16384 blocks of 256; 1 = one-shot, 8 vectors per thread (all loads
 * in flight before the stores); 2 = one-shot, 4 vectors per thread; 3 = as 0
 * over 1024 blocks. No counterpart in the reference. */
int axon_copy_shape(const void* src, void* dst, size_t bytes, int shape,
                    axon_stream_t stream);

/* Single-pass cumsum (hw variant 2 of "cumsum" and "cumsum_probs"): a chunk
 * polls each earlier chunk's published total at most `polls` times (default
 * 4096), then recomputes the missing total from the input, so the result is
 * the same for every bound, including 0 (always recompute). Process-wide;
 * applies to launches enqueued after the call. Returns the previous bound. */
uint32_t axon_scan_poll_bound(uint32_t polls);

#ifdef __cplusplus
}
#endif

#endif /* AXON_HIP_H */
