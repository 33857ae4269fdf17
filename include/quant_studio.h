/*
 * quant_studio.h -- C ABI of the MI355X (gfx950) GGUF block quantizer library
 * (libqs_hip.so). Plain pointers and sizes only; no torch or HIP types in the
 * signatures (the stream is passed as an opaque hipStream_t value).
 *
 * The reference's plugin interface for this path is the QuantSpec registry:
 *   QuantSpec(ggml_type, ftype, bytes_per_elem, needs_imatrix, make_kernel,
 *             uses_imatrix)                       kernels/common.py:27-37
 *   make_kernel(device, qw) -> quant_fn           e.g. kernels/q4_k.py:82-83
 *   quant_fn(x: f32 (n, k)) -> uint8 (n, k//blk*type_size)
 *                                                 e.g. kernels/q4_k.py:25-27
 * called once per row chunk by the pipeline (quant-studio.py:198 on the GPU,
 * :229 on the CPU). qs_quantize() replaces one quant_fn call; the imatrix
 * argument is make_kernel's qw; the bf16/f16 source is read in-kernel, which
 * replaces the pipeline's separate upcast pass (quant-studio.py:197).
 *
 * Return codes: 0 on success, a negative errno-style value on failure
 * (QS_EINVAL, QS_ENOTSUP, QS_EIO); qs_last_error() then describes it.
 */
#ifndef QUANT_STUDIO_H
#define QUANT_STUDIO_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QS_ABI_VERSION 4

#define QS_EINVAL (-22)
#define QS_ENOTSUP (-95)
#define QS_EIO (-5)

/* ggml type ids (GGUF spec) accepted as ggml_type */
#define QS_TYPE_Q4_0 2
#define QS_TYPE_Q2_K 10
#define QS_TYPE_Q3_K 11
#define QS_TYPE_Q4_K 12
#define QS_TYPE_Q5_K 13
#define QS_TYPE_Q6_K 14
#define QS_TYPE_IQ2_XXS 16
#define QS_TYPE_IQ2_XS 17
#define QS_TYPE_IQ3_XXS 18
#define QS_TYPE_IQ3_S 21
#define QS_TYPE_IQ2_S 22
#define QS_TYPE_IQ4_XS 23
/* ggml formats the reference has no quantizer for (its command line stops on
 * them, quant-studio.py:396-399); the targets of its shape fallback
 * (kernels/scheme.py:364-384) and of Q4_0/Q5_0 mixes with an imatrix
 * (scheme.py:521-523) */
#define QS_TYPE_Q4_1 3
#define QS_TYPE_Q5_0 6
#define QS_TYPE_Q5_1 7
#define QS_TYPE_Q8_0 8
#define QS_TYPE_IQ4_NL 20

/* source element types accepted as src_type (ggml ids; TORCH_DTYPES
 * kernels/common.py:20-24) */
#define QS_SRC_F32 0
#define QS_SRC_F16 1
#define QS_SRC_BF16 30

/* Version of this ABI (QS_ABI_VERSION). */
int qs_abi_version(void);

/* Upload the constant tables the quantizers read (the square-root map and
 * every IQ grid / neighbour-list table, about 7.5 MB) to `device` now, with
 * blocking copies, and keep them until the process ends. qs_quantize() does
 * the same lazily on its first call per device (and per IQ grid): a
 * hipMalloc plus a blocking hipMemcpy inside that call. Callers that must not
 * allocate or synchronise inside qs_quantize (stream capture into a graph, a
 * latency-critical loop) call qs_init() for each device first; every later
 * qs_quantize() on that device then only launches. The reference builds its
 * tables lazily per kernel module (tables_for, kernels/iq2.py:80-84,
 * iq2xs_common.py:101-106, iq3_common.py:81-85). */
int qs_init(int device);

/* Square-root rounding of the weights sqrt(sigma2 + x^2) and sqrt(w) that the
 * K-quant, IQ4 and IQ quantizers with an imatrix (and Q4_K/Q5_K without one)
 * compute. The reference takes them with torch.sqrt (e.g. kernels/q4_k.py:34,
 * :51; iq2.py:431-436), whose rounding depends on where it runs:
 *   QS_SQRT_TORCH_CPU      torch.sqrt on a CPU tensor on an Intel x86-64 host
 *                          (MKL: one ulp below the IEEE root on 98,955 of the
 *                          2^24 mantissa/parity classes), the host that wrote
 *                          the golden vectors; the default
 *   QS_SQRT_IEEE           the correctly rounded root (torch.sqrt on a GPU
 *                          tensor, as on the reference's CUDA path; C sqrtf)
 *   QS_SQRT_TORCH_CPU_AMD  torch.sqrt on a CPU tensor on an AMD EPYC host (the
 *                          MI355X machine's; MKL there: one ulp below on 7.4% and
 *                          one ulp above on 9.8% of the classes of normal
 *                          inputs, the IEEE root on every subnormal input)
 * Process-wide; read by each qs_quantize() call at launch. */
#define QS_SQRT_TORCH_CPU 0
#define QS_SQRT_IEEE 1
#define QS_SQRT_TORCH_CPU_AMD 2
int qs_set_sqrt_rounding(int mode);
int qs_get_sqrt_rounding(void);

/* 1 if ggml_type has a HIP quantizer in this build, else 0. Mirrors the
 * registry membership test `type in QUANT_TYPES` (kernels/__init__.py:18-27,
 * quant-studio.py:396-399). */
int qs_type_supported(int ggml_type);

/* 1 if the type's QuantSpec.needs_imatrix is set (kernels/common.py:33): the
 * command line refuses to plan it without an imatrix (quant-studio.py:400-406).
 * 0 if not, QS_ENOTSUP for an unknown type. qs_quantize() itself requires an
 * imatrix only for IQ2_XXS, IQ2_XS and IQ2_S, whose reference quantizers have
 * no path without one; IQ3_XXS (needs_imatrix = 1) quantizes without one as
 * quantize_iq3_xxs(x, None) does (weights x^2, iq3_xxs.py:41-42). */
int qs_type_needs_imatrix(int ggml_type);

/* 1 if the type uses an imatrix when one is given (QuantSpec.uses_imatrix,
 * kernels/common.py:36; Q4_0 ignores it, q4_0.py:36-37). */
int qs_type_uses_imatrix(int ggml_type);

/* Bytes of one quantized row of k values (k/blk * type_size, the BLOCK_BYTES
 * constants e.g. kernels/q4_k.py:19), or QS_EINVAL if k is not a multiple of
 * the block size (the precondition of every quant_fn, e.g. q4_k.py:26). */
int64_t qs_row_bytes(int ggml_type, int64_t k);

/* Quantize n_rows rows of k values (one quant_fn call, e.g. q4_k.py:25-79).
 *   src:           device pointer to the first row; 16-byte aligned
 *   src_row_stride_bytes: distance between rows, a multiple of 16, >= k*elem
 *   imatrix:       device pointer to k f32 column weights, or NULL; required
 *                  by IQ2_XXS / IQ2_XS / IQ2_S (QS_EINVAL otherwise); ignored
 *                  by Q4_0, Q4_1, Q5_0, Q5_1 and Q8_0
 *   dst:           device pointer receiving n_rows * qs_row_bytes(k) bytes;
 *                  dst_bytes must be at least that
 *   hip_stream:    hipStream_t to launch on (NULL = null stream)
 * At most 2^34 values (n_rows * k) per call, and n_rows * src_row_stride_bytes
 * below 2^62; larger calls are refused with QS_EINVAL (split them by rows).
 * Asynchronous and stream-ordered: the kernel is queued on hip_stream and the
 * call returns; the launch status is the return value (the caller's
 * hipGetLastError() state is left alone). The kernels use no device memory
 * beyond src, imatrix, dst and the constant tables; the first call per device
 * (and per IQ grid) uploads those tables (hipMalloc and a blocking copy,
 * under a process-wide lock) unless qs_init() did. Every call takes that lock
 * briefly to look the tables up. Safe to call from several threads. The output
 * bytes do not depend on how rows are split across calls. */
int qs_quantize(int ggml_type, int src_type, const void *src, int64_t n_rows, int64_t k,
                int64_t src_row_stride_bytes, const float *imatrix, void *dst,
                int64_t dst_bytes, void *hip_stream);

/* Message describing the last failure on the calling thread ("" if none). */
const char *qs_last_error(void);

/* ---- host pipeline of the command line ----
 *
 * Replaces the reference's CudaPipeline (quant-studio.py:148-213), its
 * OutputWriter (:103-131) and copy_tensor (:235-241): rows are read chunk by
 * chunk from the input file (pread, qs_pipeline_quantize_fd) or from host
 * memory (qs_pipeline_quantize) into pinned buffers, quantized on the device
 * and written with pwrite() at the tensor's offset in the output file. The caller keeps the GGUF header,
 * tensor order and offsets, the type plan and the chunk size (--mem).
 * Calls on one pipeline must not overlap; they may come from different
 * threads (the command line creates its pipeline on a thread of its own and
 * drives it from the main thread). Host memory passed in must stay valid, and
 * fd open, until qs_pipeline_finish() returns.
 */
typedef struct qs_pipeline qs_pipeline;

/* Number of visible ROCm devices (0 when there are none or HIP fails). The
 * reference's device choice tests torch.cuda.is_available() (pick_device,
 * quant-studio.py:51-58). */
int qs_device_count(void);

/* Pipeline on `device` with n_slots input slots (2..16; 3 keeps the host
 * copy, H2D and kernel of consecutive chunks overlapped), max(8, 2 n_slots)
 * output slots (device output and its pinned copy, so a writer a few chunks
 * behind does not hold back the next uploads), and n_copy_threads host
 * threads (1..64) that read or copy each chunk's rows into pinned memory. */
int qs_pipeline_create(int device, int n_slots, int n_copy_threads, qs_pipeline **out);

/* Queue one tensor: n_rows rows of k values of src_type at host address src
 * (rows contiguous), quantized to ggml_type in chunks of rows_per_chunk rows
 * with the host imatrix (k floats or NULL; as qs_quantize; copied before the
 * call returns), the output rows written contiguously at out_offset of fd.
 * The rows of each chunk are read by the pipeline's threads while the
 * previous chunk's upload and kernel are queued; the call returns
 * with its last chunk still being read (that chunk is queued by the next call
 * on the pipeline or by qs_pipeline_finish), and blocks only while all slots
 * are busy. At most 2^34 values per tensor (QS_EINVAL otherwise). One
 * pipeline.quantize_tensor call of the reference (quant-studio.py:180-213,
 * driven from :453-461). */
int qs_pipeline_quantize(qs_pipeline *p, int ggml_type, int src_type, const void *src,
                         int64_t n_rows, int64_t k, const float *imatrix,
                         int64_t rows_per_chunk, int fd, int64_t out_offset);

/* As qs_pipeline_quantize, with the rows read from the file src_fd (rows
 * contiguous from byte src_offset) with pread() instead of copied from host
 * memory. The command line passes its input GGUF this way: the copies read the
 * page cache without mapping it, so they take no page faults and the process
 * has no multi-GB mapping to tear down (unmapping 8 GB of faulted-in rows took
 * 0.04-0.12 s on the MI355X machine's host). The same pipeline.quantize_tensor
 * call of the reference (quant-studio.py:180-213, which reads the rows through
 * gguf-py's memory map). src_fd must stay open until qs_pipeline_finish()
 * returns; a read error or a file that ends inside the tensor fails this call,
 * the next one or qs_pipeline_finish with QS_EIO. */
int qs_pipeline_quantize_fd(qs_pipeline *p, int ggml_type, int src_type, int src_fd,
                            int64_t src_offset, int64_t n_rows, int64_t k, const float *imatrix,
                            int64_t rows_per_chunk, int fd, int64_t out_offset);

/* Queue a write of nbytes host bytes at out_offset of fd, in order with the
 * quantized chunks (a passthrough tensor, copy_tensor quant-studio.py:235-241). */
int qs_pipeline_write(qs_pipeline *p, const void *src, int64_t nbytes, int fd, int64_t out_offset);

/* Queue the last pending chunk and wait until everything queued is written
 * (OutputWriter.flush, quant-studio.py:128-130); returns the first failure of
 * any queued step. */
int qs_pipeline_finish(qs_pipeline *p);

/* Queue the last pending chunk and wait for queued work, then release the
 * pipeline's threads, buffers, streams and events. NULL is ignored. */
void qs_pipeline_destroy(qs_pipeline *p);

#ifdef __cplusplus
}
#endif
#endif /* QUANT_STUDIO_H */
