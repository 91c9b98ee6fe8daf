/*
 * khrt - the C-ABI boundary of the MI355X (gfx950) kernel.h runtime.
 *
 * Plain pointers and sizes only. Every function returns an int status:
 * 0 on success, otherwise a non-zero code (a hipError_t value, or one of the
 * KHRT_E_* codes below) and khrt_last_error() holds a non-empty message for
 * the calling thread. This mirrors the reference runtime's
 * Result<T> = expected<T, Error{code != 0, message != ""}> contract
 * (include/kernelh/runtime/runtime_error.hpp:20-31) across a C boundary:
 * nothing throws through this ABI.
 *
 * Layers (each group cites the reference interface it replaces):
 *   1. Backend: device, memory, module, raw launch, events
 *        include/kernelh/runtime/backend.hpp:56-96 (HipBackend,
 *        lib/runtime/backend_hip.cpp:47-245)
 *   2. Descriptor packing (2N+3 memref slots)
 *        include/kernelh/runtime/descriptor_packing.hpp:27-60
 *   3. Device limits (gfx950 entry), launch verifier, occupancy
 *        include/kernelh/compiler/device_limits.hpp:50-82,
 *        include/kernelh/compiler/launch_verifier.hpp:54-88,
 *        include/kernelh/compiler/occupancy.hpp:56-103
 *   4. Verified launch (KernelLaunch::launch)
 *        include/kernelh/runtime/kernel_launch.hpp:26-65,
 *        lib/runtime/kernel_launch.cpp:100-132
 *   5. The seven templates: embedded gfx950 code objects, launcher-owned
 *      geometry and one entry point per template (the symbols and memref
 *      argument lists of lib/dsl/kernels/<name>.cpp).
 */
#ifndef KHRT_H
#define KHRT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KHRT_API __attribute__((visibility("default")))

/* Internal status codes (hipError_t values pass through unchanged). */
#define KHRT_OK 0
#define KHRT_E_INVALID 1       /* bad argument / shape / null handle          */
#define KHRT_E_REFUSED 2       /* launch refused by the pre-launch verifier   */
#define KHRT_E_UNKNOWN_TARGET 3 /* device_limits_for: unknown target token    */
#define KHRT_E_NO_DEVICE 4     /* no HIP device / runtime unavailable         */
#define KHRT_E_SKIP 77         /* skip convention (runtime_error.hpp:15-20)   */

typedef struct khrt_dim3 {
  unsigned x, y, z;
} khrt_dim3;

/* Live device properties (backend.hpp:31-38 DeviceInfo) plus the gfx arch. */
typedef struct khrt_device_info {
  char name[256];
  char arch[64]; /* e.g. "gfx950:sramecc+:xnack-" */
  int64_t lds_bytes_per_workgroup;
  int32_t wavefront_size;
  int32_t max_threads_per_workgroup;
  int64_t cu_count;
  int64_t vram_bytes;
  int64_t max_grid_dim[3];
  int32_t clock_khz;
  int32_t memory_clock_khz;
  int32_t memory_bus_width;
  int32_t l2_bytes;
} khrt_device_info;

/* Thread-local message of the last failure ("" when none). */
KHRT_API const char *khrt_last_error(void);
/* hipGetErrorString-equivalent; safe without a device. */
KHRT_API const char *khrt_error_string(int code);
/* Library version string. */
KHRT_API const char *khrt_version(void);

/* ---- 1. Backend (backend.hpp:56-96) ------------------------------------ */
KHRT_API int khrt_device_count(int *count);
KHRT_API int khrt_init_device(int ordinal);
KHRT_API int khrt_get_device_info(khrt_device_info *out);
KHRT_API int khrt_device_synchronize(void);
/* Plain hipMalloc/hipFree and synchronous H2D/D2H copies (buffer.hpp:1-5). */
KHRT_API int khrt_malloc(void **out, size_t bytes);
KHRT_API int khrt_free(void *ptr);
KHRT_API int khrt_memcpy_h2d(void *dst, const void *src, size_t bytes);
KHRT_API int khrt_memcpy_d2h(void *dst, const void *src, size_t bytes);
KHRT_API int khrt_memcpy_d2d(void *dst, const void *src, size_t bytes);
/* Fills `count` floats with `value` by a device kernel on `stream`. */
KHRT_API int khrt_fill_f32(void *dst, float value, size_t count, void *stream);
/* Module lifecycle (gpu_module.hpp:17-42): a corrupted or truncated image
 * is a typed error, never a crash. */
KHRT_API int khrt_module_load_data(void **module, const void *image, size_t size);
/* Extent in bytes of an AMDGPU ELF64 code object, read from its own
 * headers: the end of the ELF header, both header tables and every segment
 * and section with file contents. For callers that hold an image without
 * its size, as Backend::module_load_data(const void *image) does
 * (backend.hpp:75; hipModuleLoadData takes no size either): it trusts, as
 * that loader does, that the bytes the headers name are there. Not an ELF
 * code object, malformed tables or an extent beyond 1 GiB -> KHRT_E_INVALID.
 * No device needed. */
KHRT_API int khrt_elf_image_size(const void *image, size_t *size);
KHRT_API int khrt_module_get_function(void **function, void *module, const char *name);
KHRT_API int khrt_module_unload(void *module);
/* Raw launch (Backend::launch_kernel): no verification. */
KHRT_API int khrt_launch_raw(void *function, khrt_dim3 grid, khrt_dim3 block,
                             size_t shared_bytes, void *stream, void **params);
/* Streams at the default priority. */
KHRT_API int khrt_stream_create(void **stream);
KHRT_API int khrt_stream_destroy(void *stream);
KHRT_API int khrt_stream_synchronize(void *stream);
/* Events (event_timer.hpp). */
KHRT_API int khrt_event_create(void **event);
KHRT_API int khrt_event_record(void *event, void *stream);
KHRT_API int khrt_event_synchronize(void *event);
KHRT_API int khrt_event_elapsed_ms(float *ms, void *start, void *end);
KHRT_API int khrt_event_destroy(void *event);

/* ---- 2. Descriptor packing (descriptor_packing.cpp:19-49) -------------- */
/* Slots of one rank-N memref: 2N+3. */
KHRT_API size_t khrt_memref_slot_count(int rank);
/* Writes {alloc ptr, aligned ptr, offset 0, sizes[N], row-major strides[N]}
 * to slots[0..2N+3). Returns 0, or KHRT_E_INVALID if cap is too small. */
KHRT_API int khrt_pack_memref(uint64_t *slots, size_t cap, const void *dev_ptr, int rank,
                              const int64_t *shape);
/* A scalar in the low bytes of one 8-byte slot (add_scalar_bytes). */
KHRT_API int khrt_pack_scalar(uint64_t *slot, const void *value, size_t byte_size);

/* ---- 3. Device limits / launch verifier / occupancy -------------------- */
typedef struct khrt_device_limits {
  int64_t lds_bytes_per_workgroup;
  int32_t wavefront_size;
  int32_t max_threads_per_workgroup;
  int64_t max_grid_dim[3];
  int64_t vram_bytes;
  int32_t waves_per_cu;
  int32_t reg_file_per_cu;
  int64_t cu_count;
  const char *name;
} khrt_device_limits;

/* device_limits_for (device_limits.cpp:119-133): exact token match among
 * "gfx950", "gfx1101", "sm_80". Unknown -> KHRT_E_UNKNOWN_TARGET with a
 * message naming the target and listing every known token. */
KHRT_API int khrt_device_limits_for(const char *target, khrt_device_limits *out);
/* Number of known targets and the i-th token. */
KHRT_API int khrt_device_target_count(void);
KHRT_API const char *khrt_device_target_name(int i);
/* query_cu_count (device_limits.hpp:76-82): live CU count when a device is
 * initialised, else limits->cu_count. */
KHRT_API int64_t khrt_query_cu_count(const khrt_device_limits *limits);
/* Limits of the live device: the gfx950 table entry overridden by the live
 * DeviceInfo fields (kernel_launch.cpp:34-50). */
KHRT_API int khrt_live_limits(khrt_device_limits *out);

typedef struct khrt_launch_config {
  int32_t threads_per_workgroup;
  int32_t grid_x, grid_y, grid_z;
  size_t static_shared_bytes;
} khrt_launch_config;

/* LaunchVerifier::verify (launch_verifier.cpp:109-172): the five rules (LDS,
 * max threads, wave multiple, grid extents, occupancy > 0), plus, for a loaded
 * kernel, its own workgroup-size bound (__launch_bounds__; the reference's
 * kernels carry none). Returns 0 when
 * launchable, KHRT_E_REFUSED otherwise with every violation, one per line,
 * copied into diag (NUL-terminated, truncated to cap). `function` may be NULL
 * (analytic occupancy) or a loaded kernel (vendor occupancy API). */
KHRT_API int khrt_verify_launch(const khrt_launch_config *config,
                                const khrt_device_limits *limits, void *function,
                                char *diag, size_t cap);

typedef struct khrt_occupancy_input {
  const char *kernel;
  const char *target;
  const char *config;
  int32_t vgpr_count;
  int64_t lds_bytes;
  int32_t threads_per_workgroup;
} khrt_occupancy_input;

typedef struct khrt_occupancy_report {
  int32_t vgpr_limited_waves;
  int32_t lds_limited_blocks;
  int32_t thread_limited_blocks;
  int32_t achieved_waves;
  double theoretical_pct;
  int32_t limiter; /* 0 none, 1 vgpr, 2 lds, 3 threads */
  int32_t measured_blocks;
  double measured_pct;
  char measured_note[256];
} khrt_occupancy_report;

/* occupancy_report (occupancy.cpp:124-221), pinned formulas. */
KHRT_API int khrt_compute_occupancy(const khrt_occupancy_input *input,
                                    const khrt_device_limits *limits, void *function,
                                    khrt_occupancy_report *out);

/* ---- 4. Verified launch (kernel_launch.cpp:100-132) --------------------- */
/* Refuses (KHRT_E_REFUSED, message "KernelLaunch::launch refused: ...") when
 * the verifier finds any violation against the live device limits; null
 * function or empty params -> KHRT_E_INVALID. Launches exactly the given
 * kernel, nothing before or after it. */
KHRT_API int khrt_kernel_launch(void *function, khrt_dim3 grid, khrt_dim3 block,
                                size_t shared_bytes, void *stream, void **params,
                                size_t param_count);

/* ---- 5. The seven templates --------------------------------------------- */
/* Registry: "vecadd", "gemm", "softmax", "layernorm", "scan", "scan_totals",
 * "fused_gelu", "attention" (lib/dsl/registry.cpp:23-36). */
KHRT_API int khrt_template_count(void);
KHRT_API const char *khrt_template_name(int i);
/* Embedded gfx950 code object (bare ELF, loadable by hipModuleLoadData) whose
 * extern "C" symbol equals the template name. Unknown -> KHRT_E_INVALID with
 * the registered names listed (program.cpp:27-37). */
KHRT_API int khrt_template_code_object(const char *name, const void **image, size_t *size);
/* Resource notes of the template's kernel symbol, read from the code object
 * at build time: vgpr, agpr, sgpr, LDS bytes, scratch bytes, wavefront size,
 * max flat workgroup size. */
typedef struct khrt_kernel_resources {
  int32_t vgpr_count;
  int32_t agpr_count;
  int32_t sgpr_count;
  int64_t lds_bytes;
  int64_t private_segment_bytes;
  int32_t wavefront_size;
  int32_t max_flat_workgroup_size;
} khrt_kernel_resources;
KHRT_API int khrt_template_resources(const char *name, khrt_kernel_resources *out);
/* The launcher-owned geometry for a template at a shape given as
 * "k=v,k=v" text (the CLI's --shape syntax, main.cpp:242-266). */
KHRT_API int khrt_template_geometry(const char *name, const char *shape, khrt_dim3 *grid,
                                    khrt_dim3 *block);
/* The kernel symbol the launcher runs for a template at a shape ("k=v,k=v"):
 * the template name itself or a variant in the same code object with the
 * same arguments and results (gemm_small, gemm_wide, gemm_ksplit,
 * gemm_ksplit_deep, softmax_wide, layernorm_wide). Writes a NUL-terminated name of at most cap
 * bytes. No reference counterpart: the reference compiles one symbol per
 * template and shape (emitter.cpp:733-736); callers that report resources
 * for a launch (kernelh compile --resources) need the symbol it runs. */
KHRT_API int khrt_template_launch_symbol(const char *name, const char *shape, char *out, size_t cap);
/* Loaded function handle of a template on the current device (module loaded
 * once per process from the embedded image). */
KHRT_API int khrt_template_function(const char *name, void **function);

/* GEMM candidates: the launcher's own `gemm` symbols (product = 1) followed by
 * the gfx950 tune space that `kernelh tune` evaluates, which re-prunes the
 * reference's BM/BN x BK x waves x unroll x vec space (autotuner.hpp:36-41,
 * autotuner.cpp:754-799) for wave64, MFMA 32x32 / 16x16 tiles and 160 KiB of
 * LDS. Every candidate takes the `gemm` template's 21 memref slots and is
 * correct for every shape and grid. No reference counterpart beyond that
 * space: the reference compiles one kernel per sampled config instead. */
typedef struct khrt_gemm_candidate {
  char symbol[64];
  char code_object[16];   /* embedded code object holding the symbol */
  char pipeline[16];      /* regs, lds-dma, prefetch2, persistent, ksplit, ksplit-deep */
  int32_t mfma;           /* 32: v_mfma_f32_32x32x2f32; 16: v_mfma_f32_16x16x4f32 */
  int32_t waves;          /* wave64s per workgroup */
  int32_t wave_grid_m, wave_grid_n;  /* waves along m and n (K-split: 1 x 1) */
  int32_t wave_tile_m, wave_tile_n;  /* C elements per wave */
  int32_t bm, bn, bk;     /* C tile per workgroup; K slab depth (K-split: k group) */
  int32_t unroll;         /* slabs (K-split: 32-k batches) in flight ahead of the MFMAs */
  int32_t prio;           /* waves raise their priority while issuing MFMAs */
  int32_t persistent;     /* grid = min(tiles, two per CU); workgroups loop over tiles */
  int32_t k_split;        /* the workgroup's waves split K, summed in a fixed order */
  int32_t product;        /* one of the launcher's own symbols */
} khrt_gemm_candidate;
KHRT_API int khrt_gemm_candidate_count(void);
KHRT_API int khrt_gemm_candidate_get(int i, khrt_gemm_candidate *out);
/* Launch geometry of a candidate at m x n x k (grid.x workgroups). */
KHRT_API int khrt_gemm_candidate_geometry(const char *symbol, int64_t m, int64_t n, int64_t k,
                                          khrt_dim3 *grid, khrt_dim3 *block);
/* Loaded function of a candidate on the current device. */
KHRT_API int khrt_gemm_candidate_function(const char *symbol, void **function);
/* Tune cache the GEMM launcher consults (main.cpp:1320-1420 keeps the
 * reference's cache for its own CLI only): the JSON-lines file `kernelh tune`
 * writes, keyed by khrt_tune_cache_key("gemm", "m=..,n=..,k=.."). When set,
 * kh_gemm, khrt_template_geometry and khrt_template_launch_symbol use the
 * cached best candidate for a shape that has an entry and the built-in
 * choice otherwise. NULL or "" turns it off. Until this is called the path
 * is taken from the KHRT_TUNE_CACHE environment variable (unset: off). The
 * file is read once per path set. */
KHRT_API int khrt_set_tune_cache(const char *path);
/* Cache key of a tuning run (main.cpp:1353-1358 keys it by kernel, shape and
 * device name, with sha256): FNV-1a 64 of "kernel|shape|device token", as 16
 * hex digits + NUL (cap >= 17). */
KHRT_API int khrt_tune_cache_key(const char *kernel, const char *shape, char *out, size_t cap);
/* "<marketing name> (<arch>) cu=<count>" of the current device, the device
 * part of the cache key ("AMD Instinct MI355X" when the runtime reports no
 * marketing name). */
KHRT_API int khrt_device_token(char *out, size_t cap);

/* One entry point per template. Device pointers, element counts, an optional
 * stream (NULL = default stream). Each packs the reference's memref argument
 * list (2N+3 slots per buffer, same order and ranks), computes the launcher's
 * geometry, runs the pre-launch verifier and launches through
 * hipModuleLaunchKernel; all are asynchronous on `stream`. */

/* vecadd: c = a + b, rank-1 [n] x3 (vecadd.cpp:44-89) -> 15 slots. */
KHRT_API int kh_vecadd(const float *a, const float *b, float *c, int64_t n, void *stream);
/* fused_gelu: out = gelu_tanh(1.5x + 0.5); tmp is the template's dead
 * fusion intermediate and is never touched (fused_gelu.cpp:73-160,
 * passes/fusion.cpp:331-333) -> 15 slots. */
KHRT_API int kh_fused_gelu(const float *x, float *tmp, float *out, int64_t n, void *stream);
/* softmax over the last dim of x[rows, cols] (softmax.cpp:68-165) -> 14 slots. */
KHRT_API int kh_softmax(const float *x, float *y, int64_t rows, int64_t cols, void *stream);
/* layernorm, eps 1e-5: x[rows,cols], gamma[cols], beta[cols], y[rows,cols]
 * (layernorm.cpp:58-153) -> 24 slots. */
KHRT_API int kh_layernorm(const float *x, const float *gamma, const float *beta, float *y,
                          int64_t rows, int64_t cols, void *stream);
/* scan: inclusive prefix sum of x[n] into y[n] (scan.cpp:163-341 argument
 * list: x, y, y_lo[n], totals_hi[T], totals_lo[T], T = ceil(n/256)) ->
 * 25 slots. y holds the finished result when the launch completes;
 * y_lo is not written. totals_hi/lo hold the look-back state: whatever they
 * contain before the first call (never written, zeroed, another kernel's
 * data), the kernel recognises it as not its own and starts afresh, and it
 * leaves them valid for the next call; the same holds for a raw
 * hipModuleLaunchKernel of the `scan` symbol. Calls that overlap in time on
 * the same totals buffers race. */
KHRT_API int kh_scan(const float *x, float *y, float *y_lo, float *totals_hi, float *totals_lo,
                     int64_t n, void *stream);
/* scan_totals: the reference's second pass (scan.cpp:350-453 argument list:
 * totals_hi, totals_lo, off_hi, off_lo, off_lo2 [T]; y, y_lo [n]) -> 35
 * slots. With the single-pass scan it leaves y and the totals unchanged and
 * writes each 256-block's exclusive offset (off_hi = fp32 rounding,
 * off_lo = off_lo2 = 0). */
KHRT_API int kh_scan_totals(const float *totals_hi, const float *totals_lo, float *off_hi,
                            float *off_lo, float *off_lo2, float *y, float *y_lo, int64_t n,
                            void *stream);
/* gemm: C[m,n] = A[m,k] B[k,n], fp32 row-major (gemm.cpp:116-296) -> 21 slots. */
KHRT_API int kh_gemm(const float *A, const float *B, float *C, int64_t m, int64_t n, int64_t k,
                     void *stream);
/* attention: O = softmax(Q K^T / sqrt(d)) V, non-causal, Q/K/V/O
 * [batch, heads, seq, head_dim] (attention.cpp:86-289) -> 44 slots.
 * head_dim must be 64 (attention.cpp:115-120). */
KHRT_API int kh_attention(const float *Q, const float *K, const float *V, float *O, int64_t batch,
                          int64_t heads, int64_t seq, int64_t head_dim, void *stream);
/* scan without allocating: y[n] = inclusive prefix sum of x[n], the result
 * of kh_scan, with the look-back state in a 4 MiB device array per GPU that
 * the library holds until the process ends, instead of caller totals. No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory at call time (HIP graph capture, serving loops, harnesses
 * that forbid hipMalloc). khrt_init_device sets it up on a device (array
 * address, scan module, verified launch shape); the call itself allocates
 * nothing and refuses a device not set up that way. n <= 2^31. Calls on one
 * GPU share its array: calls that overlap in time on one GPU race. */
KHRT_API int kh_scan_noalloc(const float *x, float *y, int64_t n, void *stream);

/* ---- 6. Roofline microbenchmarks (bench/refs/roofline.hip:22-53,
 *         bench/harness/roofline.cpp:60-130) ------------------------------ */
/* c = a + b over n floats (n a multiple of 4, 16-byte aligned buffers):
 * the measured HBM ceiling when 12 n bytes exceed the 256 MB MALL. */
KHRT_API int kh_roofline_triad(const float *a, const float *b, float *c, int64_t n, void *stream);
/* dst = src over n floats (n a multiple of 4, 16-byte aligned): a kernel of
 * exactly known traffic (4n B read, 4n B written) for counter calibration. */
KHRT_API int kh_roofline_copy(const float *src, float *dst, int64_t n, void *stream);
/* fp32 MFMA rate: `blocks` workgroups of 256 threads each run `iters`
 * rounds of 8 independent v_mfma_f32_32x32x2f32 per wave. FLOPs executed =
 * blocks * 4 * iters * 8 * 4096. out needs blocks * 256 floats. */
KHRT_API int kh_roofline_mfma(float *out, int64_t blocks, int64_t iters, void *stream);

/* ---- 7. Bench metrics (bench/harness/metrics.cpp:5-52) ------------------ */
/* One of the reference's metric formulas by name, with its arguments in
 * order: gflops_from_ms and gbps_from_ms (work, ms); gemm_flops and
 * gemm_bytes (m, n, k); elementwise_bytes and layernorm_bytes (rows, cols);
 * scan_bytes, fused_gelu_bytes and roofline_triad_bytes (n);
 * attention_flops (batch, heads, seq, head_dim); roofline_fma_flops (fmas).
 * KHRT_E_INVALID for an unknown name or a wrong argument count. */
KHRT_API int khrt_bench_metric(const char *formula, const double *args, int nargs, double *out);
/* The work of one `kernelh bench` row by those formulas: bytes (*is_flops =
 * 0) or FLOPs (1) per launch of `kernel` (vecadd, fused_gelu, softmax,
 * layernorm, scan, gemm, attention, roofline_triad) at `shape`. vecadd
 * counts as the triad (three streams of n floats). The rows' rate column is
 * work * 1000 / ms / 1e9. */
KHRT_API int khrt_bench_row_work(const char *kernel, const char *shape, double *work, int *is_flops);

#ifdef __cplusplus
}
#endif

#endif /* KHRT_H */
