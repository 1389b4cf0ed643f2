/*
 * grpo_hip.h -- C ABI of libgrpo_hip.so, the MI355X (gfx950) kernels of the
 * GRPO rollout decode step.
 *
 * Every pointer argument is a DEVICE pointer owned by the caller (torch); the
 * library never allocates device memory.  Scratch space is passed in
 * explicitly ("workspace").  Every entry point is asynchronous on the given
 * stream (a hipStream_t passed as void*; NULL = the default stream) and makes
 * no host synchronisation.  bf16 tensors are passed as void* (2-byte
 * bfloat16 elements).
 *
 * Return codes: 0 = success; < 0 = invalid argument (the Python layer raises
 * ValueError, matching the reference's shape/dtype checks); > 0 = a HIP
 * runtime error code (RuntimeError).  grpo_last_error() returns a
 * thread-local message describing the last failure.
 */
#ifndef GRPO_HIP_H
#define GRPO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* grpo_stream_t;

#define GRPO_OK 0
#define GRPO_EINVAL (-1)
#define GRPO_EUNSUPPORTED (-2)
#define GRPO_EWORKSPACE (-3)

/* Library/ABI version (major*10000 + minor*100 + patch). */
int grpo_version(void);

/* Checks that a gfx950 device is present and current.  0 if usable.
 * Python raises ImportError when this fails (the reference raises ImportError
 * when its kernel backend is unavailable: src/triton_kernels/__init__.py:297). */
int grpo_init(void);

/* Thread-local description of the last error returned on this thread. */
const char* grpo_last_error(void);

/* ------------------------------------------------------------------ NF4 --
 * NF4 dequantization, bit-exact.  Replaces the dequant half of
 * _lora_forward_kernel (src/triton_kernels/lora_forward.py:171-206) and
 * bitsandbytes.functional.dequantize_4bit (src/core/lora.py:39-47) for
 * non-nested quant states.
 *   w       : packed nibbles, ceil(numel/2) bytes; element e is the high nibble
 *             of byte e/2 when e is even, the low nibble when e is odd
 *   absmax  : float32 [ceil(numel/blocksize)]
 *   code16  : float32 [16] codebook (quant_state.code)
 *   out     : bf16 [numel], out[e] = bf16_rne(code16[q_e] * absmax[e/blocksize])
 */
int grpo_nf4_dequant(const uint8_t* w, const float* absmax, const float* code16, void* out,
                     int64_t numel, int blocksize, grpo_stream_t stream);

/* Workspace bytes grpo_nf4_lora_linear needs for this shape (0 if none).
 * Layout: the first 64 KiB hold split-K group counters, the rest partial sums.
 * The counters must be zero before the first use (zero-fill a new workspace
 * once); every call leaves them at zero, so one workspace can serve calls of
 * any shape in stream order.  Calls that may run concurrently must not share a
 * workspace, and the workspace must not be used for anything else. */
size_t grpo_nf4_lora_linear_workspace_bytes(int M, int N, int K, int r);

/* y[M,N] = bf16(bf16(bf16(x W^T) + bias) + bf16(bf16(bf16(x A^T) B^T) * bf16(scaling)))
 * -- the fused NF4 + LoRA forward of FusedLoRAFunction.forward /
 * _lora_forward_kernel (src/triton_kernels/lora_forward.py:653-759, 107-260).
 *   x       : bf16 [M, K], row stride ldx (elements)
 *   w/absmax/code16/blocksize : non-nested NF4 weight of logical shape [N, K]
 *   bias    : bf16 [N] or NULL
 *   lora_a  : bf16 [r, K] (row-major), lora_b: bf16 [N, r]; r == 0 drops the
 *             LoRA term (plain NF4 linear; lora_a/lora_b may be NULL)
 *   y       : bf16 [M, N], row stride ldy
 */
int grpo_nf4_lora_linear(const void* x, int64_t ldx, const uint8_t* w, const float* absmax,
                         const float* code16, int blocksize, const void* bias, const void* lora_a,
                         const void* lora_b, int r, float scaling, void* y, int64_t ldy, int M,
                         int N, int K, void* workspace, size_t workspace_bytes,
                         grpo_stream_t stream);

/* ------------------------------------------------------------ paged KV --
 * Cache layout: k_cache, v_cache bf16 [num_blocks, Hkv, block_size, D],
 * contiguous.  block_tables int32 [B, max_blocks] (row stride bt_stride),
 * context_lens int32 [B]; both device-resident and read-only to the kernels.
 *
 * KV append: writes k_new[b,h,:], v_new[b,h,:] (bf16 [B, Hkv, D], strides in
 * elements, last dim contiguous) at slot context_lens[b] (the pre-increment
 * length) of sequence b.  Replaces _paged_kv_update_kernel
 * (src/triton_kernels/paged_kv.py:253-319), GQA-native (H = Hkv).  Rows whose
 * slot lies outside the table or whose block id is outside [0, num_blocks)
 * are skipped. */
int grpo_paged_kv_append(const void* k_new, const void* v_new, int64_t kn_stride_b,
                         int64_t kn_stride_h, void* k_cache, void* v_cache, int64_t num_blocks,
                         const int32_t* block_tables, int64_t bt_stride,
                         const int32_t* context_lens, int B, int Hkv, int D, int block_size,
                         int max_blocks, grpo_stream_t stream);

/* Workspace bytes of grpo_paged_attn_decode for this shape (0 if none). */
size_t grpo_paged_attn_workspace_bytes(int B, int Hq, int Hkv, int D, int block_size,
                                       int max_blocks);

/* Single-query paged decode attention with GQA: for every sequence b and query
 * head h, out[b,h,:] = sum_t softmax_t(scale * q[b,h].k_t) v_t over
 * t < context_lens[b], with k_t/v_t from KV head h / (Hq/Hkv); denominator
 * max(sum, 1e-6); context_lens[b] == 0 gives zeros.  Replaces
 * _paged_attention_decode_kernel (src/triton_kernels/paged_kv.py:63-251).
 *   q       : bf16 [B, Hq, D], strides q_stride_b/q_stride_h (elements)
 *   out     : [B, Hq, D] contiguous, float32 (out_bf16 == 0, the reference's
 *             output dtype) or bf16 rounded RNE (out_bf16 != 0)
 *   workspace: grpo_paged_attn_workspace_bytes(...) bytes, no initialisation
 *             needed */
int grpo_paged_attn_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                           const void* k_cache, const void* v_cache, int64_t num_blocks,
                           const int32_t* block_tables, int64_t bt_stride,
                           const int32_t* context_lens, void* out, int out_bf16, int B, int Hq,
                           int Hkv, int D, int block_size, int max_blocks, float scale,
                           void* workspace, size_t workspace_bytes, grpo_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* GRPO_HIP_H */
