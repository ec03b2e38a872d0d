/*
 * kapel_hip.h -- C ABI of libkapel_hip.so, the MI355X (gfx950) implementation
 * of Kapel's product by quantized weights (`kapel_ops::QuantizedMatmul`).
 *
 * Plain pointers and sizes only.  Device pointers are HIP device addresses;
 * `stream` is a hipStream_t passed as a pointer (NULL: the null stream).
 * Every call is asynchronous on `stream` and returns a status code; no call
 * aborts or throws across this boundary.
 *
 * Reference interfaces replaced (paths under crates/ of smallbard/kapel):
 *   codes            kapel-cuda-abi/src/lib.rs:152-194 (float and quant codes)
 *   kh_qmatmul       kapel-ops/src/matmul.rs:89-156 (QuantizedMatmul::infer),
 *                    kapel-cuda/src/quantized.rs:73-224 (Cuda::quantized_product),
 *                    kapel-cpu/src/matmul.rs:263-311 (Run<QuantizedMatmul> for Cpu),
 *                    kernels/src/lib.rs:3207 (qgemv), :4061-4128 (qgemv_<fmt>)
 *   kh_quantize_x    kapel-cpu/src/bytes.rs:110-158 (activations to bytes)
 *   kh_block_dots    kapel-cpu/src/bytes.rs:356-394 (the i32 block dots)
 *   kh_dequantize    kernels/src/lib.rs:3745-3766 (dequantize)
 *   kh_dequantize_rows kernels/src/lib.rs:3773-3792 (dequantize_rows),
 *                    kapel-cuda/src/quantized.rs:358-386
 *   kh_expert_matmul kapel-ops/src/experts.rs:130-229 (ExpertMatmul),
 *                    kapel-cuda/src/experts.rs:127-250, kernels/src/lib.rs:3507-3681
 *                    (expert_gemv, expert_gemv_bytes)
 *   kh_quantize_host kapel-core/src/dtype.rs:751-782 (quantize)
 *   kh_block_len/... kapel-core/src/dtype.rs:140-213
 */
#ifndef KAPEL_HIP_H
#define KAPEL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Quantized formats: kapel-cuda-abi/src/lib.rs:167-194, plus Q2_K and Q3_K,
 * which have no code there. */
#define KH_INT8 0u
#define KH_INT4 1u
#define KH_Q8_0 2u
#define KH_Q4_0 3u
#define KH_Q4_1 4u
#define KH_Q5_0 5u
#define KH_Q5_1 6u
#define KH_Q4K 7u
#define KH_Q5K 8u
#define KH_Q6K 9u
#define KH_IQ4_NL 10u /* f32 activations only (bytes.rs:51-77 has no IQ) */
#define KH_IQ4_XS 11u
#define KH_IQ3_S 12u
#define KH_Q2K 13u
#define KH_Q3K 14u

/* Float types: kapel-cuda-abi/src/lib.rs:152-163 (the 8-bit ones are not
 * taken by this library). */
#define KH_F32 0u
#define KH_BF16 1u
#define KH_F16 2u

/* Status codes: the refusals of QuantizedMatmul::infer
 * (kapel-ops/src/matmul.rs:105-150) and of the launch
 * (kapel-cuda/src/device.rs:673-718). */
#define KH_OK 0
#define KH_ERR_ARITY 1         /* Error::Arity: no weights */
#define KH_ERR_DTYPE 2         /* Error::UnsupportedDType: format or float code */
#define KH_ERR_SHAPE 3         /* Error::InvalidArgument: sizes disagree */
#define KH_ERR_MISALIGNED 4    /* Error::BlockMisaligned: K not whole blocks */
#define KH_ERR_OVERFLOW 5      /* Error::Overflow: a size beyond the kernels' range */
#define KH_ERR_WORKSPACE 6     /* workspace missing or too small */
#define KH_ERR_HIP 7           /* a HIP runtime error */
#define KH_ERR_NULL 8          /* a required pointer is NULL */

/* Flags of kh_qmatmul. */
/* Activations quantized to bytes by blocks of 32 (kapel-cpu/src/bytes.rs),
 * integer block dots; taken only if every weight's format is read that way
 * (bytes.rs:51-77) and x has at most 16 rows, as Cpu::with_byte_activations
 * (kapel-cpu/src/matmul.rs:14,292-306: above IN_PLACE_ROWS = 16 rows the CPU
 * multiplies dequantized f32 tiles, and so does this library). */
#define KH_BYTE_ACTIVATIONS 1u
/* The activations were prepared in this workspace by the previous call with
 * the same x, rows, k and mode: the call goes straight to the products (for
 * one x multiplied by weights given in several calls). */
#define KH_REUSE_ACTIVATIONS 2u
/* Byte activations at every row count (batched decode and prefill in
 * bytes, the int8 MFMA product): as KH_BYTE_ACTIVATIONS without its 16-row
 * limit.  A divergence from kapel-cpu, whose products above 16 rows are f32
 * whatever the mode; it has no counterpart in the reference. */
#define KH_BYTE_ACTIVATIONS_ALL_ROWS 4u

/* One weight matrix of a product: n rows of k elements, `bytes` bytes of
 * blocks at `data` (device), the rows stacked after those of the previous
 * weights (kapel-ops/src/matmul.rs:94-98). */
typedef struct kh_weight {
    uint32_t format; /* KH_INT8 ... KH_Q3K */
    uint32_t group;  /* elements per group of Kapel's int8/int4; 0 otherwise */
    const void *data;
    uint64_t bytes;  /* n * row bytes */
    uint64_t n;
} kh_weight;

/* Library identity: a NUL-terminated string. */
const char *kh_version(void);
/* Text of a status code. */
const char *kh_error_string(int status);

/* kapel-core/src/dtype.rs:140-187: elements and bytes of a block; 0 for a
 * format or group that does not exist. */
uint32_t kh_block_len(uint32_t format, uint32_t group);
uint32_t kh_block_bytes(uint32_t format, uint32_t group);

/* Bytes of workspace kh_qmatmul needs for these arguments. */
uint64_t kh_qmatmul_workspace(const kh_weight *weights, uint32_t count, uint64_t k,
                              uint64_t rows, uint32_t flags);

/* out [rows, sum n] = x [rows, k] . [w_1; w_2; ...]^T, out in `out_kind`
 * (the activations' type, as the op's signature says).  x and out are
 * contiguous device arrays; weight data 4-byte aligned.  `workspace`
 * (device, kh_qmatmul_workspace bytes, 256-byte aligned) must be zero-filled
 * before its first use; every call leaves it in a
 * state the next call accepts.  Calls that share a workspace must be ordered
 * (one stream).  Results are bitwise the same from run to run: every
 * reduction is split by the shapes only.
 * Replaces: QuantizedMatmul (kapel-ops/src/matmul.rs:89-156) with
 * Cuda::quantized_product (kapel-cuda/src/quantized.rs:73-224). */
int kh_qmatmul(const kh_weight *weights, uint32_t count, uint64_t k, uint32_t x_kind,
               const void *x, uint64_t rows, uint32_t out_kind, void *out, uint32_t flags,
               void *workspace, uint64_t workspace_bytes, void *stream);

/* kh_qmatmul without a workspace argument, for callers that cannot allocate
 * (code under graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  The scratch is a
 * file-scope device array of KH_STATIC_SCRATCH_BYTES on each device, held
 * until the process ends; a call whose kh_qmatmul_workspace exceeds it is
 * refused with KH_ERR_WORKSPACE before anything is launched.  It calls no
 * hipMalloc or hipFree; the first call on a device clears the array's
 * counters on its stream.  Every call on one device shares that device's
 * array: calls that overlap on one device (two streams, two host threads)
 * race, so they must be ordered; KH_REUSE_ACTIVATIONS reuses what the
 * previous call on the device left in it. */
#define KH_STATIC_SCRATCH_BYTES (32ull << 20)
int kh_qmatmul_static(const kh_weight *weights, uint32_t count, uint64_t k, uint32_t x_kind,
                      const void *x, uint64_t rows, uint32_t out_kind, void *out, uint32_t flags,
                      void *stream);

/* Activations in bytes (kapel-cpu/src/bytes.rs:144-158): for each block of
 * 32, scale = max|x| / 127 and q = round-half-even(x * 127 / max) in
 * [-127, 127]; sums32 = scale * (sum of q).  q [rows, k] i8, scale and
 * sums32 [rows, k/32] f32 (device).  k must be a multiple of 32. */
int kh_quantize_x(uint32_t x_kind, const void *x, uint64_t rows, uint64_t k, int8_t *q,
                  float *scale, float *sums32, void *stream);

/* The i32 block dots of the byte-activation product of one weight matrix
 * (kapel-cpu/src/bytes.rs:356-394): dots [rows, n, k/16]; the dot of a group
 * of 32 at the slot of its first element / 16, the other slot 0; a group of
 * 16 (Q6_K) at its own slot.  Codes as bytes.rs:282-353 decodes them (Q6_K
 * signed, the others as stored).  Exposed to check the integers bit for bit;
 * the product computes the same integers in the same kernels. */
int kh_block_dots(const kh_weight *weight, uint64_t k, const int8_t *q, uint64_t rows,
                  int32_t *dots, void *workspace, uint64_t workspace_bytes, void *stream);

/* Rows first .. first + count of a weight, dequantized to `out_kind`
 * (kernels/src/lib.rs:3745-3766): out [count, k]. */
int kh_dequantize(const kh_weight *weight, uint64_t k, uint64_t first, uint64_t count,
                  uint32_t out_kind, void *out, void *stream);

/* Gathered rows of a quantized table (kernels/src/lib.rs:3773-3792):
 * out [count, k] = dequantized rows indices[0..count] (u32, device). */
int kh_dequantize_rows(const kh_weight *weight, uint64_t k, const uint32_t *indices,
                       uint64_t count, uint32_t out_kind, void *out, void *stream);

/* The product of each token by its experts (mixtures of experts).  weight:
 * the experts' matrices stacked, [experts * n, k] (expert e: rows e n ..
 * (e + 1) n); x [tokens, k] (per_route 0) or [tokens, topk, k] (per_route
 * 1), contiguous on the device; idx [tokens * topk] u32 on the device, each
 * token's experts; out [tokens, topk, n] in `out_kind`:
 *     out[t, j, i] = sum_c x[t, (j,) c] w[idx[t, j] n + i, c].
 * An index of `experts` or more gives NaN outputs for its route (the device
 * never faults; kernels/src/lib.rs:3499-3504).  Flags: KH_BYTE_ACTIVATIONS
 * as for kh_qmatmul.  The workspace (kh_expert_matmul_workspace bytes,
 * 256-byte aligned) is used only when x is not 16-byte aligned (f32) or
 * 8-byte aligned (16-bit).
 * Replaces: ExpertMatmul (kapel-ops/src/experts.rs:130-229) with
 * Cuda's expert_gemv / expert_gemv_bytes (kapel-cuda/src/experts.rs:127-250,
 * kernels/src/lib.rs:3507-3681). */
uint64_t kh_expert_matmul_workspace(const kh_weight *weight, uint32_t experts, uint64_t k,
                                    uint64_t tokens, uint32_t topk, uint32_t per_route,
                                    uint32_t x_kind, uint32_t flags);
int kh_expert_matmul(const kh_weight *weight, uint32_t experts, uint64_t k, uint32_t x_kind,
                     const void *x, uint64_t tokens, uint32_t topk, uint32_t per_route,
                     const uint32_t *idx, uint32_t out_kind, void *out, uint32_t flags,
                     void *workspace, uint64_t workspace_bytes, void *stream);

/* Host quantization at load time (kapel-core/src/dtype.rs:751-782 for int8,
 * int4, Q8_0, Q4_0, Q4_1, by the reference's rules; Q5_0, Q5_1, Q2_K, Q3_K,
 * Q4_K, Q5_K and Q6_K by this library's round-to-nearest encoders, which the
 * reference does not have).  values [count] f32 host, count a multiple of
 * the block; out host, count / block_len * block_bytes bytes.  `threads` <= 1
 * runs on the calling thread.  Returns bytes written, or a negative status. */
int64_t kh_quantize_host(uint32_t format, uint32_t group, const float *values, uint64_t count,
                         uint8_t *out, int threads);

#ifdef __cplusplus
}
#endif

#endif /* KAPEL_HIP_H */
