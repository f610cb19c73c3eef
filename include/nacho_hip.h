/*
 * nacho_hip.h — C ABI of the MI355X (gfx950) backend for nacho's GPU target.
 *
 * Each GPU kernel that the reference declares for the operations this backend covers
 * (csr_add, csr_add_3, csr_mul, coo_add, coo_mul, coo3d_add, csf_add, dcsr_add, dcsr_mul,
 * dcsr_mul_without_recursive_partitioning, spgemm, sssmm, coo_csr_add, inner_prod,
 * inner_prod_coo: compiler.cpp:112-153) gets one extern "C" entry point here.  The reference binds
 * `namespace <k> { Z_tensor_format <k>_gpu_i32_f32(a, b, num_blocks, threads_per_block); }`
 * (entry point printed at src/backend/stitch_and_generate.cpp:299-301,
 * called from the wrapper written by src/backend/generate_bindings.cpp:288-314).  These
 * functions replace those generated entry points: same operands, same meaning of every
 * field, same launch-geometry arguments, plus an explicit stream and an optional allocator.
 *
 * Tensor descriptors are plain C structs whose field order is the reference's generated
 * tensor struct (src/backend/tensor.cpp:13-61: dimension sizes first, then the level arrays
 * in level order, then `values`, then `nnz`).  Index arrays are int32, values float32, all
 * pointers are device pointers except where stated.
 *
 * Return value of every entry point: 0 on success, a positive hipError_t value when a HIP
 * call failed, or one of the negative NACHO_ERR_* codes.  On failure every scratch buffer is
 * released and the result descriptor is left zeroed.  nacho_error_string() names a code.
 *
 * Ownership: operands are borrowed and never written.  Result buffers are allocated by
 * `alloc` (or by the library's caching device allocator when `alloc` is NULL, in which case
 * the caller releases them with nacho_free()).  A result array of length 0 is a NULL pointer.
 *
 * Ordering: an entry point returns once the result lengths are known; the last kernels that
 * fill the result arrays may still be running on `stream`.  Work the caller queues on the
 * same stream sees complete results; other streams must wait for `stream` (an event), and
 * host reads must synchronise it, as with any stream-ordered library.  The reference's
 * generated entry point likewise returns after launching its write pass.
 *
 * Input contract (the reference's, made explicit): pos[0] == 0, pos non-decreasing,
 * pos[rows] == length of the coordinate array, coordinates strictly increasing within
 * each fibre (sorted, no duplicates), COO/COO3 coordinates sorted lexicographically and
 * distinct.  As in the reference, the entry points do not check it on the device: host-side
 * shape and pointer checks return NACHO_ERR_INVALID_ARGUMENT, operand contents are trusted,
 * and nacho_validate_csr() checks a CSR operand on request.
 */
#ifndef NACHO_HIP_H
#define NACHO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- error codes ------------------------------------------------------------------- */
#define NACHO_OK 0
#define NACHO_ERR_INVALID_ARGUMENT (-1) /* null pointer, negative size, shape mismatch   */
#define NACHO_ERR_INDEX_OVERFLOW (-2)   /* result or work count does not fit int32        */
#define NACHO_ERR_OUT_OF_MEMORY (-3)    /* the allocator returned NULL                    */
#define NACHO_ERR_MALFORMED_INPUT (-4)  /* nacho_validate_* found unsorted/duplicate/bad
                                           pos, or a reader found a malformed file     */
#define NACHO_ERR_NO_DEVICE (-5)        /* no HIP device visible                          */
#define NACHO_ERR_INTERNAL (-6)         /* a kernel did not publish a result length       */
#define NACHO_ERR_IO (-7)               /* a file could not be opened or read             */
#define NACHO_ERR_UNSUPPORTED (-8)      /* a file format variant the reader does not take */
#define NACHO_ERR_SCRATCH_TOO_SMALL (-9) /* input beyond an allocation-free entry point's
                                            static scratch (NACHO_NOALLOC_MAX_ITEMS)     */

/* ---- tensor descriptors (field order = the reference's generated structs) ---------- */

/* CSR, format {i: Dense, j: Compressed_unique} named "CSR" (compiler.cpp:21-24).
 * Reference struct: {dim_i_size, dim_j_size, dim_j_offsets, dim_j_length, dim_j_indices,
 * values, nnz} (tensor.cpp:13-61). */
typedef struct nacho_csr {
    int32_t dim_i_size;     /* rows                                              */
    int32_t dim_j_size;     /* columns                                           */
    int32_t *dim_j_offsets; /* pos, dim_i_size + 1 entries                       */
    int32_t dim_j_length;   /* number of stored coordinates                      */
    int32_t *dim_j_indices; /* crd, dim_j_length entries                         */
    float *values;          /* dim_j_length entries                              */
    int32_t nnz;            /* == dim_j_length                                   */
} nacho_csr;

/* CSR whose offsets are 64-bit: the SpGEMM result, whose length can exceed 2^31.  Same
 * field order as nacho_csr; no counterpart in the reference, which is int32-only
 * (index_t = int32_t, stitch_and_generate.cpp:235). */
typedef struct nacho_csr64 {
    int32_t dim_i_size;
    int32_t dim_j_size;
    int64_t *dim_j_offsets; /* dim_i_size + 1 entries */
    int64_t dim_j_length;
    int32_t *dim_j_indices;
    float *values;
    int64_t nnz;
} nacho_csr64;

/* COO, format {i: Compressed_non_unique, j: Singleton_unique} named "COO"
 * (compiler.cpp:50-53), lowered to one merged level (Compile.cpp:66-154).  Reference struct:
 * {dim_i_size, dim_j_size, dim_i_length, dim_i_indices, dim_j_length, dim_j_indices, values,
 * nnz}. */
typedef struct nacho_coo {
    int32_t dim_i_size;
    int32_t dim_j_size;
    int32_t dim_i_length;
    int32_t *dim_i_indices;
    int32_t dim_j_length;
    int32_t *dim_j_indices;
    float *values;
    int32_t nnz;
} nacho_coo;

/* COO3, format {i: Compressed_non_unique, j: Singleton_non_unique, k: Singleton_unique}
 * named "COO3" (compiler.cpp:60-64). */
typedef struct nacho_coo3 {
    int32_t dim_i_size;
    int32_t dim_j_size;
    int32_t dim_k_size;
    int32_t dim_i_length;
    int32_t *dim_i_indices;
    int32_t dim_j_length;
    int32_t *dim_j_indices;
    int32_t dim_k_length;
    int32_t *dim_k_indices;
    float *values;
    int32_t nnz;
} nacho_coo3;

/* DCSR, format {i, j: Compressed_unique} named "DCSR" (compiler.cpp:39-42): rows are
 * compressed too, so only rows with entries are stored (nacho.to_dcsr drops empty rows,
 * python/nacho/convert.py:34-53).  The outermost compressed level has no offsets
 * (tensor.cpp:36-39). */
typedef struct nacho_dcsr {
    int32_t dim_i_size;
    int32_t dim_j_size;
    int32_t dim_i_length;   /* stored rows                 */
    int32_t *dim_i_indices; /* dim_i_length row ids        */
    int32_t *dim_j_offsets; /* dim_i_length + 1 entries    */
    int32_t dim_j_length;
    int32_t *dim_j_indices; /* dim_j_length entries        */
    float *values;          /* dim_j_length entries        */
    int32_t nnz;
} nacho_dcsr;

/* CSF3, format {i, j, k: Compressed_unique} named "CSF3" (compiler.cpp:44-48).  The
 * outermost compressed level has no offsets (tensor.cpp:36-39). */
typedef struct nacho_csf3 {
    int32_t dim_i_size;
    int32_t dim_j_size;
    int32_t dim_k_size;
    int32_t dim_i_length;
    int32_t *dim_i_indices; /* dim_i_length entries       */
    int32_t *dim_j_offsets; /* dim_i_length + 1 entries   */
    int32_t dim_j_length;
    int32_t *dim_j_indices; /* dim_j_length entries       */
    int32_t *dim_k_offsets; /* dim_j_length + 1 entries   */
    int32_t dim_k_length;
    int32_t *dim_k_indices; /* dim_k_length entries       */
    float *values;          /* dim_k_length entries       */
    int32_t nnz;
} nacho_csf3;

/* Scalar, format {} named "Scalar" (compiler.cpp:75): the single value of a full
 * reduction.  Reference struct: {values, nnz} (tensor.cpp:13-61 with no levels; the values
 * buffer holds one element). */
typedef struct nacho_scalar {
    float *values; /* 1 entry */
    int32_t nnz;   /* 1       */
} nacho_scalar;

/* ---- allocation ------------------------------------------------------------------- */

/* Caller-supplied device allocator, used for results and scratch.  `allocate` returns NULL
 * on failure.  `stream` is the hipStream_t the call runs on.  `release` is called for
 * scratch buffers when the entry point returns, possibly while kernels queued on `stream`
 * still use them: it must be stream-ordered (reuse only by work queued later on `stream`,
 * or after synchronising it), like hipFreeAsync or torch's caching allocator.  Replaces the generated code's
 * cudaMallocAsync/cudaFreeAsync on stream 0 (stitch_and_generate_gpu.cpp:187-196) and the
 * Python deleter of runtime/nacho_nb.h:50-58. */
typedef struct nacho_allocator {
    void *ctx;
    void *(*allocate)(void *ctx, size_t bytes, void *stream);
    void (*release)(void *ctx, void *ptr, void *stream);
} nacho_allocator;

/* Release a buffer that an entry point allocated with the default allocator (alloc == NULL).
 * Stream-ordered on `stream`.  Replaces cudaFreeWrapper (runtime/cuda_utils/cuda_utils.cu:7-11). */
int nacho_free(void *ptr, void *stream);

/* The default allocator keeps freed buffers cached for reuse by later calls (per size class,
 * stream-ordered).  This returns every cached, unused buffer to the driver. */
int nacho_release_cached_memory(void);

/* Cap on the bytes the default allocator keeps cached (unused buffers held for reuse);
 * SIZE_MAX, the default, keeps every released buffer.  A release that takes the cache past
 * the cap synchronises the device and returns the oldest buffers of the largest sizes to
 * the driver until it fits; setting a cap trims at once.  No counterpart in the reference
 * (cudaMallocAsync's pool, stitch_and_generate_gpu.cpp:187-196). */
int nacho_set_cache_limit(size_t bytes);

/* Bytes the default allocator holds cached (released, unused) now. */
size_t nacho_cached_bytes(void);

/* Note that work queued on `stream` uses the buffer `ptr` (a buffer the default allocator
 * returned, not yet released).  When the buffer is released on its own stream, an event is
 * also recorded on `stream`, and the buffer is reused only by work ordered after it: a
 * consumer on another stream may drop its reference before its reads finish.  The
 * counterpart of torch's Tensor.record_stream for this library's buffers; the reference,
 * which runs everything on stream 0, has none.  NACHO_ERR_INVALID_ARGUMENT if `ptr` is not
 * a live buffer of the default allocator. */
int nacho_record_stream(void *ptr, void *stream);

/* ---- entry points ------------------------------------------------------------------
 * `num_blocks` / `threads_per_block` are the reference's launch arguments
 * (generate_bindings.cpp:292-325, default 256/256).  They are accepted and validated
 * (both > 0) but advisory: the gfx950 kernels pick their own tiles.
 * `stream` is a hipStream_t (NULL = the null stream, as the reference's `stream = 0`). */

/* Z = a + b over CSR (union; explicit zeros kept).  Replaces csr_add::csr_add_gpu_i32_f32
 * (kernel declared at compiler.cpp:112). */
int nacho_gpu_csr_add_f32(const nacho_csr *a, const nacho_csr *b, nacho_csr *z,
                          int32_t num_blocks, int32_t threads_per_block, void *stream,
                          const nacho_allocator *alloc);

/* Allocation-free Z = a + b over CSR: the same result as nacho_gpu_csr_add_f32, computed
 * without allocating anything (no hipMalloc / hipFree / allocating library routine).  No
 * counterpart in the reference; for callers that cannot allocate: code that must not call
 * hipMalloc (serving loops, harnesses that forbid it, work prepared for HIP graph capture).
 *   - The caller passes the result buffers in `z`: dim_j_offsets (dim_i_size + 1 entries),
 *     dim_j_indices and values, each with room for z->dim_j_length entries, which must be
 *     at least a->dim_j_length + b->dim_j_length (the union's upper bound).  On return
 *     z->dim_j_length and z->nnz hold the result length (0 on failure); the pointers are
 *     left as given.
 *   - Scratch is a static device array of 8 MiB per GPU (held until the process ends),
 *     enough for a->dim_j_length + b->dim_j_length + dim_i_size <= NACHO_NOALLOC_MAX_ITEMS;
 *     larger inputs fail with NACHO_ERR_SCRATCH_TOO_SMALL before any device work.
 *   - Every call on a GPU shares that GPU's scratch, so calls on one GPU take turns: a
 *     call holds a per-GPU lock from its first launch until its kernels have finished
 *     (it synchronises `stream` before returning, also on failure), so calls from other
 *     host threads wait, and no kernel of a returned call still reads the scratch when
 *     the next call, on any stream, starts.  The scratch keeps the last call's contents;
 *     each call clears what must start at zero.
 *   - The call synchronises `stream` to read the result length back. */
#define NACHO_NOALLOC_MAX_ITEMS 250000000LL
int nacho_gpu_csr_add_f32_noalloc(const nacho_csr *a, const nacho_csr *b, nacho_csr *z,
                                  int32_t num_blocks, int32_t threads_per_block,
                                  void *stream);

/* Z = a + b + c over CSR (union of three; a value is the sum of the present operands in
 * the order (a + b) + c, one float32 add per extra operand).  Replaces
 * csr_add_3::csr_add_3_gpu_i32_f32 (compiler.cpp:114). */
int nacho_gpu_csr_add_3_f32(const nacho_csr *a, const nacho_csr *b, const nacho_csr *c,
                            nacho_csr *z, int32_t num_blocks, int32_t threads_per_block,
                            void *stream, const nacho_allocator *alloc);

/* Z = a * b elementwise over CSR (intersection).  Replaces csr_mul::csr_mul_gpu_i32_f32
 * (compiler.cpp:116), including its empty-result early exit
 * (stitch_and_generate.cpp:168-220): an empty product returns zeroed offsets and NULL
 * coordinate/value arrays. */
int nacho_gpu_csr_mul_f32(const nacho_csr *a, const nacho_csr *b, nacho_csr *z,
                          int32_t num_blocks, int32_t threads_per_block, void *stream,
                          const nacho_allocator *alloc);

/* Z = a + b over COO (union of (i, j) tuples).  Replaces coo_add::coo_add_gpu_i32_f32
 * (compiler.cpp:118). */
int nacho_gpu_coo_add_f32(const nacho_coo *a, const nacho_coo *b, nacho_coo *z,
                          int32_t num_blocks, int32_t threads_per_block, void *stream,
                          const nacho_allocator *alloc);

/* Z = a * b over COO (intersection of (i, j) tuples).  Replaces coo_mul::coo_mul_gpu_i32_f32
 * (compiler.cpp:120). */
int nacho_gpu_coo_mul_f32(const nacho_coo *a, const nacho_coo *b, nacho_coo *z,
                          int32_t num_blocks, int32_t threads_per_block, void *stream,
                          const nacho_allocator *alloc);

/* Z = a + b over COO3 (union of (i, j, k) tuples).  Replaces
 * coo3d_add::coo3d_add_gpu_i32_f32 (compiler.cpp:138). */
int nacho_gpu_coo3d_add_f32(const nacho_coo3 *a, const nacho_coo3 *b, nacho_coo3 *z,
                            int32_t num_blocks, int32_t threads_per_block, void *stream,
                            const nacho_allocator *alloc);

/* Z = a + b with a CSR left operand and a COO right operand, giving CSR (union; a + b where
 * both hold a coordinate, explicit zeros kept).  The COO operand must be sorted by (i, j)
 * without duplicates, as nacho.to_coo builds it.  Replaces coo_csr_add::coo_csr_add_gpu_i32_f32
 * (kernel declared at compiler.cpp:122). */
int nacho_gpu_coo_csr_add_f32(const nacho_csr *a, const nacho_coo *b, nacho_csr *z,
                              int32_t num_blocks, int32_t threads_per_block, void *stream,
                              const nacho_allocator *alloc);

/* z = sum_ijk a_ijk * b_ijk over CSF3 operands: the inner product, a Scalar.  Each product
 * is one float32 multiply (as the reference's a * b); the products are summed in float64
 * in a fixed order (deterministic run to run) and rounded once, where the reference adds
 * float32 partial sums with atomics (compute.cpp:498-520, nacho_kernel_utils.h:40-58).
 * Replaces inner_prod::inner_prod_gpu_i32_f32 (compiler.cpp:141).  Asynchronous: the value
 * is ready when `stream` reaches the end of the call's work. */
int nacho_gpu_inner_prod_f32(const nacho_csf3 *a, const nacho_csf3 *b, nacho_scalar *z,
                             int32_t num_blocks, int32_t threads_per_block, void *stream,
                             const nacho_allocator *alloc);

/* The same inner product over COO3 operands (sorted by (i, j, k), no duplicates).
 * Replaces inner_prod_coo::inner_prod_coo_gpu_i32_f32 (compiler.cpp:143). */
int nacho_gpu_inner_prod_coo_f32(const nacho_coo3 *a, const nacho_coo3 *b, nacho_scalar *z,
                                 int32_t num_blocks, int32_t threads_per_block, void *stream,
                                 const nacho_allocator *alloc);

/* Z = a + b over CSF3 (union at every level; every coordinate of each level's union is
 * emitted).  Replaces csf_add::csf_add_gpu_i32_f32 (compiler.cpp:135). */
int nacho_gpu_csf_add_f32(const nacho_csf3 *a, const nacho_csf3 *b, nacho_csf3 *z,
                          int32_t num_blocks, int32_t threads_per_block, void *stream,
                          const nacho_allocator *alloc);

/* Z = a + b over DCSR (union of row ids, then of each row's columns).  Replaces
 * dcsr_add::dcsr_add_gpu_i32_f32 (compiler.cpp:124). */
int nacho_gpu_dcsr_add_f32(const nacho_dcsr *a, const nacho_dcsr *b, nacho_dcsr *z,
                           int32_t num_blocks, int32_t threads_per_block, void *stream,
                           const nacho_allocator *alloc);

/* Z = a * b elementwise over DCSR.  The result's rows are the row ids stored in both
 * operands, each with the intersection of its columns (possibly empty: the generated code
 * emits the row at its i lattice point whatever the inner level yields, compute.cpp:945-990).
 * Replaces dcsr_mul::dcsr_mul_gpu_i32_f32 (compiler.cpp:126). */
int nacho_gpu_dcsr_mul_f32(const nacho_dcsr *a, const nacho_dcsr *b, nacho_dcsr *z,
                           int32_t num_blocks, int32_t threads_per_block, void *stream,
                           const nacho_allocator *alloc);

/* The same product as nacho_gpu_dcsr_mul_f32.  Replaces
 * dcsr_mul_without_recursive_partitioning (compiler.cpp:128-133), which differs from
 * dcsr_mul only in how the reference partitions work; the result is identical. */
int nacho_gpu_dcsr_mul_without_recursive_partitioning_f32(
    const nacho_dcsr *a, const nacho_dcsr *b, nacho_dcsr *z, int32_t num_blocks,
    int32_t threads_per_block, void *stream, const nacho_allocator *alloc);

/* Masked SpGEMM: Z_ik = sum_j a_ij * b_jk * c_ik for the (i, k) stored in c that at least
 * one product a_ij * b_jk reaches (Z's pattern = c's pattern intersected with a*b's).  Each
 * term is ((a * b) * c) in float32; an entry's terms are summed in float64 and rounded
 * once.  Replaces sssmm::sssmm_gpu_i32_f32 (compiler.cpp:150-153, GPU-only). */
int nacho_gpu_sssmm_f32(const nacho_csr *a, const nacho_csr *b, const nacho_csr *c,
                        nacho_csr *z, int32_t num_blocks, int32_t threads_per_block,
                        void *stream, const nacho_allocator *alloc);

/* Z_ik = sum_j a_ij * b_jk over CSR operands (ESC SpGEMM), int32 result.  Replaces
 * spgemm::spgemm_gpu_i32_f32 (compiler.cpp:145-148).  Fails with NACHO_ERR_INDEX_OVERFLOW
 * when nnz(Z) does not fit int32; use nacho_gpu_spgemm64_f32 then. */
int nacho_gpu_spgemm_f32(const nacho_csr *a, const nacho_csr *b, nacho_csr *z,
                         int32_t num_blocks, int32_t threads_per_block, void *stream,
                         const nacho_allocator *alloc);

/* The same product with 64-bit result offsets and 64-bit product counts, for results and
 * intermediate product counts beyond 2^31 (the R-MAT scale-20 square has 6.0e9 products and
 * 3.6e9 result entries).  No counterpart in the reference (int32-only). */
int nacho_gpu_spgemm64_f32(const nacho_csr *a, const nacho_csr *b, nacho_csr64 *z,
                           int32_t num_blocks, int32_t threads_per_block, void *stream,
                           const nacho_allocator *alloc);

/* ---- input validation ------------------------------------------------------------
 * The entry points trust operand contents, as the reference's generated code does.  This
 * checks a CSR operand against the input contract on the device: pos[0] == 0, pos
 * non-decreasing, pos[rows] == dim_j_length, 0 <= crd < dim_j_size, crd strictly
 * increasing within each row.  Returns NACHO_OK, NACHO_ERR_MALFORMED_INPUT, or
 * NACHO_ERR_INVALID_ARGUMENT for host-visible faults (null pointers, negative sizes).
 * Synchronises `stream`.  No counterpart in the reference (its generated code checks
 * nothing). */
int nacho_validate_csr(const nacho_csr *t, void *stream);

/* ---- file readers (host) ---------------------------------------------------------
 * Matrix Market and FROSTT readers, replacing nacho.parse2D / nacho.parse3D_i32_f32
 * (runtime/io/parse.h:28-263, registered at runtime/register_runtime.cpp:20-40).  Arrays are
 * host memory allocated by the library; release each with nacho_host_free(). */

/* Coordinates and values of a Matrix Market file, in file order (0-based). */
typedef struct nacho_coo2d_host {
    int32_t N;      /* rows    */
    int32_t M;      /* columns */
    int64_t nnz;    /* entries, including mirrored ones of symmetric files */
    int32_t *row;
    int32_t *col;
    float *data;
} nacho_coo2d_host;

/* Coordinates and values of a FROSTT .tns file, in file order (0-based). */
typedef struct nacho_coo3d_host {
    int32_t N, M, K;
    int64_t nnz;
    int32_t *row;
    int32_t *col;
    int32_t *dep;
    float *data;
} nacho_coo3d_host;

/* parse2D: a `coordinate real` Matrix Market file with general, symmetric or
 * skew-symmetric symmetry.  Symmetric files get the mirror of every off-diagonal entry
 * appended after the file's entries (negated when skew-symmetric), as the reference does.
 * Values are read as double and rounded to float.  Returns NACHO_ERR_IO,
 * NACHO_ERR_UNSUPPORTED (another field or symmetry) or NACHO_ERR_MALFORMED_INPUT where the
 * reference terminates the process. */
int nacho_parse2d(const char *path, nacho_coo2d_host *out);

/* parse3D_i32_f32: "i j k value" lines (1-based) of a tensor of shape (N, M, K), read up
 * to the first entry that does not parse; values are read as float. */
int nacho_parse3d(const char *path, int32_t N, int32_t M, int32_t K, nacho_coo3d_host *out);

/* Release an array returned by a reader. */
void nacho_host_free(void *p);

/* ---- diagnostics ------------------------------------------------------------------ */

/* Static string naming an error code (HIP codes use hipGetErrorString). */
const char *nacho_error_string(int code);

/* Copy `bytes` (a multiple of 16, both pointers 16-byte aligned) from device memory `src`
 * to `dst` on `stream` with the library's own streaming copy kernel: the bandwidth reference
 * a roofline measurement states beside the peak.  Returns NACHO_ERR_INVALID_ARGUMENT for
 * misaligned or null buffers.  No counterpart in the reference. */
int nacho_device_copy(void *dst, const void *src, size_t bytes, void *stream);

/* Library version string. */
const char *nacho_version(void);

/* When enabled (nonzero), every entry point brackets its dominant kernel with HIP events
 * on its stream, and nacho_last_kernel_ms() returns that kernel's duration for the most
 * recent call on this host thread (0 when disabled). */
void nacho_set_kernel_timing(int enable);
float nacho_last_kernel_ms(void);

/* Name of the kernel nacho_last_kernel_ms() timed in the last call on this thread. */
const char *nacho_last_kernel_name(void);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* NACHO_HIP_H */
