/*
 * grpo_hip.h -- C ABI of libgrpo_hip.so, the MI355X (gfx950) kernels of the
 * GRPO rollout decode step.
 *
 * Every pointer argument is a DEVICE pointer owned by the caller (torch); the
 * library never allocates device memory.  Scratch space is passed in
 * explicitly ("workspace" arguments, grpo_linear_parts_t buffers).  Every
 * entry point is asynchronous on the given stream (a hipStream_t passed as
 * void*; NULL = the default stream) and makes no host synchronisation.  bf16
 * tensors are passed as void* (2-byte bfloat16 elements).
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

/* Float32 absmax of a double-quantized (nested) NF4 state, for the kernels
 * above: out[i] = fma(code2[absmax_q[i]], absmax2[i / bs2], offset) in one
 * rounding, as the reference's kernel computes it (lora_forward.py:187-199,
 * whose multiply-add the compiler contracts).  absmax_q uint8 [n_blocks];
 * code2 float32 [256]; absmax2 float32 [ceil(n_blocks / bs2)]. */
int grpo_nf4_absmax_expand(const uint8_t* absmax_q, const float* code2, const float* absmax2,
                           int bs2, float offset, int64_t n_blocks, float* out,
                           grpo_stream_t stream);

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
/* The same in float16: out[e] = float16_rne(code16[q_e] * absmax[e/blocksize]),
 * the weight as the reference casts it for float16 gradients
 * (_lora_grad_x_base_kernel, lora_forward.py:343). */
int grpo_nf4_dequant_f16(const uint8_t* w, const float* absmax, const float* code16, void* out,
                         int64_t numel, int blocksize, grpo_stream_t stream);

/* Input gradient of the NF4 linear (training side of the fused NF4 + LoRA
 * linear): out[m, k] = bf16(sum_n grad[m, n] * W[n, k]) with W =
 * bf16_rne(code16[q] * absmax) as in grpo_nf4_dequant and float32
 * accumulation; with addend != NULL, out = bf16(out + addend[m, k]).
 * Replaces _lora_grad_x_base_kernel (src/triton_kernels/lora_forward.py:
 * 262-348) and the `grad_x_base + grad_x_lora` add of
 * FusedLoRAFunction.backward (:873).
 *   grad   : bf16 [M, N], row stride ldg (elements, multiple of 8), 16-byte aligned
 *   w      : packed NF4 [N * K / 2] bytes (W[N, K] row-major, even element =
 *            high nibble), 4-byte aligned; absmax float32 [N * K / blocksize]
 *   addend : bf16 [M, K] (row stride ld_add) or NULL
 *   out    : bf16 [M, K] (row stride ldo)
 * N % 32 == 0, K % 128 == 0, blocksize % 8 == 0. */
int grpo_nf4_grad_x(const void* grad, int64_t ldg, const uint8_t* w, const float* absmax,
                    const float* code16, int blocksize, int M, int N, int K, const void* addend,
                    int64_t ld_add, void* out, int64_t ldo, grpo_stream_t stream);

/* ------------------------------------------------ split-K NF4 linear --
 * The fast NF4 (+ LoRA) linear runs as a split-K kernel: workgroups own a
 * 16-row tile of W and one slice of K, so every CU gets work even when N/16
 * is small, and they write float32 partial sums.  The reduction over slices
 * (fixed order, deterministic) and the reference's rounding points
 * (lora_forward.py:243-257) are applied by the kernel that consumes the
 * result: grpo_nf4_linear_finish for a bf16 output, or the fused consumers of
 * the decode step (grpo_add_rmsnorm_parts, grpo_qkv_rope_append_parts,
 * grpo_silu_mul_parts).
 *
 * Output rows [seg_end[s-1], seg_end[s]) form segment s (one segment for a
 * plain projection; q|k|v or gate|up stacked in one weight), each with its own
 * bias, LoRA A [r, K] and LoRA B [rows_s, r]. */
#define GRPO_MAX_SEGMENTS 4

typedef struct grpo_linear_parts {
  float* part;   /* float32 [splits][M][N]: per-slice partial sums of x W^T   */
  float* tpart;  /* float32 [splits][nseg][M][16]: partial sums of x A_s^T, r > 0 */
  int splits;    /* slices of K, from grpo_nf4_linear_plan                     */
  int M, N, K, nseg, r;
  int seg_end[GRPO_MAX_SEGMENTS];         /* exclusive end row of each segment */
  const void* bias[GRPO_MAX_SEGMENTS];    /* bf16 [rows_s] or NULL             */
  const void* lora_b[GRPO_MAX_SEGMENTS];  /* bf16 [rows_s, r] when r > 0       */
  float scaling;                          /* LoRA alpha / r                    */
} grpo_linear_parts_t;

/* Launch plan of the split-K path for this shape: number of K slices and the
 * bytes of part/tpart.  GRPO_OK if the path supports the shape (M <= 64,
 * K % 256 == 0, N % 16 == 0, segment ends % 16 == 0, r <= 16, power-of-two
 * blocksize >= 64), GRPO_EUNSUPPORTED otherwise. */
int grpo_nf4_linear_plan(int M, int N, int K, int r, int nseg, int blocksize, int* splits,
                         size_t* part_bytes, size_t* tpart_bytes);

/* Partial sums of one NF4 (+ LoRA) linear into parts->part / parts->tpart
 * (parts->splits must be the planned value).  x: bf16 [M, K], row stride ldx
 * (a multiple of 8); w/absmax/code16/blocksize: non-nested NF4 weight of
 * logical shape [N, K]; lora_a: HOST array of nseg device pointers to bf16
 * [r, K] (ignored when r == 0).  The dequant-matmul half of
 * _lora_forward_kernel (lora_forward.py:107-241). */
int grpo_nf4_linear_partials(const void* x, int64_t ldx, const uint8_t* w, const float* absmax,
                             const float* code16, int blocksize, const void* const* lora_a,
                             const grpo_linear_parts_t* parts, grpo_stream_t stream);

/* y[M, N] (bf16, row stride ldy) from partial sums: the epilogue of
 * _lora_forward_kernel, y = bf16(bf16(bf16(acc) + bias) + bf16(bf16(bf16(t) B^T)
 * * bf16(scaling))) with acc, t summed over slices in slice order. */
int grpo_nf4_linear_finish(const grpo_linear_parts_t* parts, void* y, int64_t ldy,
                           grpo_stream_t stream);

/* ---- one-launch NF4 (+ LoRA) linear for decode batches (M <= 32) --------
 *
 * The fused forward of _lora_forward_kernel (lora_forward.py:107-260) with
 * its epilogue, finished in ONE launch without partial sums: one workgroup
 * per 16 output columns takes the whole of K (its waves split the k-steps and
 * meet in LDS), stages all of x in LDS and multiplies it by the segment's
 * LoRA A itself.  Same roundings as grpo_nf4_linear_finish:
 * y = bf16(bf16(bf16(acc) + bias) + bf16(bf16(bf16(t) B^T) * bf16(scaling))).
 * Shapes: M <= 32, N % 16 == 0, K % 256 == 0 with x [M, K] (+ 32 KiB per 16
 * waves) within 160 KiB of LDS, segment ends multiples of 16, r <= 16,
 * power-of-two blocksize >= 64 (grpo_nf4_tile_supported).  Up to 8 rows with
 * K % 512 == 0 take 8 columns per workgroup (K folded into the MFMA's idle
 * rows), otherwise 16.  lora_a / lora_b / bias are DEVICE pointers here;
 * lora_a in the packed order of grpo_nf4_tile_pack_lora_a. */
typedef struct grpo_tile_linear {
  int M, N, K, nseg, r;
  int seg_end[GRPO_MAX_SEGMENTS];         /* exclusive end row of each segment */
  const void* lora_a[GRPO_MAX_SEGMENTS];  /* packed LoRA A when r > 0          */
  const void* lora_b[GRPO_MAX_SEGMENTS];  /* bf16 [rows_s, r] when r > 0       */
  const void* bias[GRPO_MAX_SEGMENTS];    /* bf16 [rows_s] or NULL             */
  float scaling;                          /* LoRA alpha / r                    */
  /* Optional (one segment, r > 0): x A^T given as float32 partial sums
   * lora_t[m][q][16], q < lora_t_parts <= 4, which the kernel adds in order
   * and rounds to bf16 instead of computing x A^T (lora_a unused): the
   * attention of the decode step leaves them for o_proj
   * (grpo_paged_attn_decode_qkv_merged). */
  const float* lora_t;
  int lora_t_parts;
} grpo_tile_linear_t;

/* 1 if the one-launch linear takes this shape, else 0 (_norm: with the
 * RMSNorm source of grpo_nf4_tile_linear_norm, which also stages the norm
 * weight in LDS). */
int grpo_nf4_tile_supported(int M, int N, int K, int r, int nseg, int blocksize);
int grpo_nf4_tile_norm_supported(int M, int N, int K, int r, int nseg, int blocksize);

/* Column groups per row of the sumsq that grpo_nf4_tile_linear_residual
 * writes for this shape (N / 8 or N / 16), 0 if the shape is not taken. */
int grpo_nf4_tile_sumsq_groups(int M, int N, int K, int r, int blocksize);

/* LoRA A [r <= 16, K] (bf16, row stride lda % 8 == 0, 16-byte aligned) in the
 * order the one-launch linear reads it: for k-step s = k / 256 and j =
 * (k % 64) / 8, the 16-byte B operands of one MFMA, lane = rank + 16 ((k %
 * 256) / 64), are one contiguous KiB, 8 elements per lane in the decode8
 * order [0,2,4,6,1,3,5,7], ranks >= r zero.  out: 16-byte aligned,
 * grpo_nf4_tile_packed_lora_a_bytes(K) bytes.  A is frozen while it is used
 * packed: repack after every update (the decode engine packs once per
 * rollout). */
size_t grpo_nf4_tile_packed_lora_a_bytes(int K);
int grpo_nf4_tile_pack_lora_a(const void* lora_a, int r, int K, int64_t lda, void* out,
                              grpo_stream_t stream);

/* y[M, N] (bf16, row stride ldy) = the finished linear of x (bf16 [M, K], row
 * stride ldx % 8 == 0, 16-byte aligned). */
int grpo_nf4_tile_linear(const void* x, int64_t ldx, const uint8_t* w, const float* absmax,
                         const float* code16, int blocksize, const grpo_tile_linear_t* lin,
                         void* y, int64_t ldy, grpo_stream_t stream);

/* grpo_nf4_tile_linear with x = RMSNorm(h) = bf16(bf16(h * inv) * norm_weight),
 * inv = 1 / sqrt(sum_g sumsq[m, g] / K + eps) (groups: a multiple of 4, <= 256
 * partial sums of h^2 per row, as grpo_nf4_linear_residual /
 * grpo_embedding_sumsq / grpo_nf4_tile_linear_residual write them; sumsq rows
 * and norm_weight 16-byte aligned): the q|k|v projection of _step with the
 * layer's input norm (paged_kv.py:712-724). */
int grpo_nf4_tile_linear_norm(const void* h, int64_t ldh, const float* sumsq, int groups,
                              const void* norm_weight, float eps, const uint8_t* w,
                              const float* absmax, const float* code16, int blocksize,
                              const grpo_tile_linear_t* lin, void* y, int64_t ldy,
                              grpo_stream_t stream);

/* grpo_nf4_tile_linear followed by the decoder layer's residual add:
 * h_out[m, n] = bf16(residual[m, n] + y[m, n]) (residual may alias h_out; row
 * stride ld), and sumsq[m, g] = sum of h_out[m, n]^2 over the columns of
 * group g (G = grpo_nf4_tile_sumsq_groups per row, N / G consecutive columns
 * each) for the next RMSNorm: o_proj and the residual of _step
 * (paged_kv.py:762-798). */
int grpo_nf4_tile_linear_residual(const void* x, int64_t ldx, const uint8_t* w,
                                  const float* absmax, const float* code16, int blocksize,
                                  const grpo_tile_linear_t* lin, const void* residual,
                                  void* h_out, int64_t ld, float* sumsq, grpo_stream_t stream);

/* Workspace bytes of grpo_nf4_lora_linear[_grouped] for this shape (0 when
 * the shape takes the workspace-free generic kernel). */
size_t grpo_nf4_lora_linear_workspace_bytes(int M, int N, int K, int r, int nseg, int blocksize);

/* y[M,N] = bf16(bf16(bf16(x W^T) + bias) + bf16(bf16(bf16(x A^T) B^T) * bf16(scaling)))
 * -- the fused NF4 + LoRA forward of FusedLoRAFunction.forward /
 * _lora_forward_kernel (src/triton_kernels/lora_forward.py:653-759, 107-260).
 *   x       : bf16 [M, K], row stride ldx (elements)
 *   w/absmax/code16/blocksize : non-nested NF4 weight of logical shape [N, K]
 *   bias    : bf16 [N] or NULL
 *   lora_a  : bf16 [r, K] (row-major), lora_b: bf16 [N, r]; r == 0 drops the
 *             LoRA term (plain NF4 linear; lora_a/lora_b may be NULL)
 *   y       : bf16 [M, N], row stride ldy
 *   workspace: grpo_nf4_lora_linear_workspace_bytes(...) bytes (no
 *             initialisation needed); two launches (partials + finish).
 * Shapes outside the split-K path (M > 64) take the NF4 GEMM
 * (grpo_nf4_gemm below; no workspace), and shapes outside both a
 * one-thread-per-output kernel with the same arithmetic. */
int grpo_nf4_lora_linear(const void* x, int64_t ldx, const uint8_t* w, const float* absmax,
                         const float* code16, int blocksize, const void* bias, const void* lora_a,
                         const void* lora_b, int r, float scaling, void* y, int64_t ldy, int M,
                         int N, int K, void* workspace, size_t workspace_bytes,
                         grpo_stream_t stream);

/* NF4 (+ bias, + LoRA) linear for batches of more than 64 rows: one MFMA GEMM
 * launch, the weight decoded in registers, the reference epilogue in the
 * kernel -- _lora_forward_kernel for any M (src/triton_kernels/lora_forward.py:
 * 107-260, the forward of FusedLoRAFunction :653-759).  Same arguments and
 * result as grpo_nf4_lora_linear, no workspace.  Requires K % 32 == 0, r <= 32,
 * a power-of-two blocksize >= 32, x rows and w (and lora_a) 16-byte aligned
 * (ldx % 8 == 0); any M and N.  grpo_nf4_gemm_supported: 1 if the shape is
 * taken (alignment aside), else 0. */
int grpo_nf4_gemm_supported(int M, int N, int K, int r, int blocksize);
int grpo_nf4_gemm(const void* x, int64_t ldx, const uint8_t* w, const float* absmax,
                  const float* code16, int blocksize, const void* bias, const void* lora_a,
                  const void* lora_b, int r, float scaling, void* y, int64_t ldy, int M, int N,
                  int K, grpo_stream_t stream);
/* grpo_nf4_gemm in float16: x, lora_a, lora_b, bias and y float16, the weight
 * values float16_rne(code * absmax), every rounding point float16 -- the
 * reference kernel with X_DTYPE = LORA_DTYPE = float16 (lora_forward.py:
 * 141-143, 745-749).  Any M (no K split). */
int grpo_nf4_gemm_f16(const void* x, int64_t ldx, const uint8_t* w, const float* absmax,
                      const float* code16, int blocksize, const void* bias, const void* lora_a,
                      const void* lora_b, int r, float scaling, void* y, int64_t ldy, int M, int N,
                      int K, grpo_stream_t stream);

/* Grouped form: the output rows are split into nseg (1..4) consecutive
 * segments of seg_rows[s] rows, stacked in ONE NF4 weight (w/absmax cover all
 * rows) and one output y[M, sum(seg_rows)].  Segment s has its own bias[s]
 * (or NULL), lora_a[s] [r, K] and lora_b[s] [seg_rows[s], r]; bias, lora_a
 * and lora_b are HOST arrays of nseg device pointers (bias itself may be
 * NULL).  One call computes what the reference computes with one
 * lora_fused_forward per projection -- the q/k/v projections of
 * fused_qkv_rope (src/triton_kernels/fused_ops.py:198-219) or gate/up of
 * fused_mlp (fused_ops.py:184-193). */
int grpo_nf4_lora_linear_grouped(const void* x, int64_t ldx, const uint8_t* w,
                                 const float* absmax, const float* code16, int blocksize, int nseg,
                                 const int* seg_rows, const void* const* bias,
                                 const void* const* lora_a, const void* const* lora_b, int r,
                                 float scaling, void* y, int64_t ldy, int M, int K,
                                 void* workspace, size_t workspace_bytes, grpo_stream_t stream);

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

/* grpo_paged_attn_decode in one launch on the fast path (D = 128, block 16,
 * Hq / Hkv <= 8, 16-byte aligned q, caches and out): the context split of each
 * (sequence, KV head) that arrives last merges the pair's splits in the kernel
 * (the order and formula of the merge launch: out bit-identical to
 * grpo_paged_attn_decode), in float32 or bf16 as out_bf16 says.  Replaces
 * _paged_attention_decode_kernel (src/triton_kernels/paged_kv.py:63-251), which
 * is one launch.  The hand-over runs through an int32 counter per pair
 * (counters: grpo_paged_attn_merge_counter_bytes(B, Hkv) bytes, 128-byte
 * aligned, ZERO before the first call and left zero by every call; calls that
 * share them must be ordered on one stream) and relies on the pair's splits
 * running on one XCD; every arrival checks its XCD and sets *xcd_err = 1 when a
 * pair's splits did not share one (that call's output is then invalid; the
 * caller checks the word after a batch of calls).  Other shapes run the one
 * generic launch of grpo_paged_attn_decode (counters unused). */
int grpo_paged_attn_decode_merged(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                  const void* k_cache, const void* v_cache, int64_t num_blocks,
                                  const int32_t* block_tables, int64_t bt_stride,
                                  const int32_t* context_lens, void* out, int out_bf16, int B,
                                  int Hq, int Hkv, int D, int block_size, int max_blocks,
                                  float scale, void* workspace, size_t workspace_bytes,
                                  int* counters, int* xcd_err, grpo_stream_t stream);

/* Merge of the split partials grpo_paged_attn_decode_qkv left in
 * attn_workspace (same B, Hq, Hkv, D, block_size, max_blocks and
 * context_lens) into out [B, Hq, D] (float32, or bf16 when out_bf16 != 0):
 * out = sum_s 2^(m_s - M) O_s / max(sum_s 2^(m_s - M) l_s, 1e-6), the
 * normalisation of _paged_attention_decode_kernel
 * (src/triton_kernels/paged_kv.py:243-251).  For wide batches, whose o_proj
 * then reads the merged bf16 rows instead of merging the splits while staging. */
int grpo_paged_attn_merge(const void* attn_workspace, const int32_t* context_lens, int B, int Hq,
                          int Hkv, int D, int block_size, int max_blocks, void* out, int out_bf16,
                          grpo_stream_t stream);

/* Allocation-free variant of grpo_paged_attn_decode: no counterpart in the
 * reference.  For callers that cannot allocate device memory or pass a
 * workspace (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments, kernels and results as
 * grpo_paged_attn_decode without workspace/workspace_bytes: the split partials
 * live in a library-owned device array of grpo_paged_attn_noalloc_max_bytes()
 * bytes per GPU (8 MiB), held until the process ends.  Shapes whose
 * grpo_paged_attn_workspace_bytes(...) exceeds it return GRPO_EWORKSPACE.  It
 * calls no allocator.  All calls on one GPU share that array: calls that
 * overlap on one GPU (two streams, two host threads) race and must be
 * serialised by the caller. */
size_t grpo_paged_attn_noalloc_max_bytes(void);
int grpo_paged_attn_decode_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                   const void* k_cache, const void* v_cache, int64_t num_blocks,
                                   const int32_t* block_tables, int64_t bt_stride,
                                   const int32_t* context_lens, void* out, int out_bf16, int B,
                                   int Hq, int Hkv, int D, int block_size, int max_blocks,
                                   float scale, grpo_stream_t stream);

/* Decode-step attention: grpo_paged_attn_decode with q, k and v taken from the
 * split-K partial sums of the q|k|v projection (finished here with its bias and
 * LoRA epilogue), RoPE applied to q and k at position append_pos[b] (cos/sin
 * tables bf16 [max_pos, D]), and the new token's K/V appended at slot
 * append_pos[b] (skipped when < 0) before attention reads the cache.
 * context_lens[b] is the attention length (0 = inactive row).  Writes split
 * partials to the workspace (grpo_paged_attn_workspace_bytes(B = qkv->M, ...))
 * for grpo_nf4_linear_partials_attn, which merges them.  Fuses fused_qkv_rope
 * (fused_ops.py:198-219), the KV update (paged_kv.py:253-319) and the
 * attention kernel (paged_kv.py:63-251) of one layer of _step
 * (paged_kv.py:712-761).  Needs D = 128, block size 16, Hq/Hkv <= 8. */
int grpo_paged_attn_decode_qkv(const grpo_linear_parts_t* qkv, int Hq, int Hkv, int D,
                               const void* cos_table, const void* sin_table, int max_pos,
                               const int32_t* append_pos, const int32_t* context_lens,
                               void* k_cache, void* v_cache, int64_t num_blocks,
                               const int32_t* block_tables, int64_t bt_stride, int block_size,
                               int max_blocks, float scale, void* workspace,
                               size_t workspace_bytes, void* out, grpo_stream_t stream);

/* grpo_paged_attn_decode_qkv that also merges its context splits: the split
 * of each (sequence, KV head) pair that finishes last combines the pair's
 * split partials (the normalisation of paged_kv.py:243-251) and writes the
 * bf16 attention output out [B, Hq * D] (8-byte aligned), which o_proj reads
 * as plain rows; a pair whose context fits one split writes it directly.
 * With o_lora_r > 0 the same step leaves the LoRA-A product of o_proj's input
 * in o_lora_t: float32 [B][Hkv][16], part kvh = sum over the pair's heads of
 * out[b, k] * o_lora_a[r][k] (o_lora_a: bf16 [o_lora_r, Hq * D], 8-byte
 * aligned), for grpo_tile_linear_t.lora_t.
 * The hand-over runs through an L2 atomic counter per pair (counters: int32
 * of grpo_paged_attn_merge_counter_bytes(B, Hkv), ZERO before the first call,
 * left zero by every call) and relies on the pair's splits running on one
 * XCD (they are launched with linear ids equal modulo 8); every arrival checks
 * its XCD, and *xcd_err becomes 1 (else left as it is) when a pair's splits
 * ran on two XCDs.  The caller checks that *xcd_err is 0 and the counters are
 * zero after a run, or the outputs of that run are not valid.  Calls sharing
 * the counters must not overlap. */
size_t grpo_paged_attn_merge_counter_bytes(int B, int Hkv);
int grpo_paged_attn_decode_qkv_merged(const grpo_linear_parts_t* qkv, int Hq, int Hkv, int D,
                                      const void* cos_table, const void* sin_table, int max_pos,
                                      const int32_t* append_pos, const int32_t* context_lens,
                                      void* k_cache, void* v_cache, int64_t num_blocks,
                                      const int32_t* block_tables, int64_t bt_stride,
                                      int block_size, int max_blocks, float scale,
                                      void* workspace, size_t workspace_bytes, int* counters,
                                      int* xcd_err, void* out, const void* o_lora_a,
                                      int o_lora_r, float* o_lora_t, grpo_stream_t stream);

/* Most K slices of the q|k|v partial sums that grpo_paged_attn_decode_qkv[_merged]
 * reads (parts->splits above it returns GRPO_EUNSUPPORTED: finish q|k|v with
 * grpo_qkv_rope_append_parts and run grpo_paged_attn_decode instead). */
int grpo_paged_attn_qkv_max_slices(void);

/* Context splits per (sequence, KV head) that grpo_paged_attn_decode[_qkv]
 * plans for this shape (0 off the fast path).  When it is 1, the out argument
 * of grpo_paged_attn_decode_qkv (bf16 [B, Hq * D], 8-byte aligned; NULL
 * otherwise) receives the normalised attention output directly and no split
 * partials are written. */
int grpo_paged_attn_splits(int B, int Hq, int Hkv, int D, int block_size, int max_blocks);

/* grpo_nf4_linear_partials with x = the attention output left by
 * grpo_paged_attn_decode_qkv in attn_workspace (x[b, h*D + d], merged over
 * context splits and rounded to bf16 while the kernel stages it): the o_proj
 * of _step (paged_kv.py:762-775).  Hq, Hkv, D, block_size, max_blocks and
 * context_lens must be those of the attention call; parts->K = Hq * D. */
int grpo_nf4_linear_partials_attn(const void* attn_workspace, const int32_t* context_lens,
                                  int Hq, int Hkv, int D, int block_size, int max_blocks,
                                  const uint8_t* w, const float* absmax, const float* code16,
                                  int blocksize, const void* const* lora_a,
                                  const grpo_linear_parts_t* parts, grpo_stream_t stream);

/* grpo_nf4_linear_partials_attn followed by grpo_linear_finish_residual in one
 * launch: the o_proj of _step and the decoder layer's residual add after it
 * (paged_kv.py:762-775, 791-798), h_out = bf16(residual + y) with y the
 * finished o_proj output (bias, LoRA: the epilogue of grpo_nf4_linear_finish,
 * same roundings), and sumsq[m, g] = sum of h_out[m, n]^2 over the 64 columns
 * of group g (G = grpo_nf4_linear_attn_residual_groups(...) per row) for the
 * post-attention RMSNorm that grpo_nf4_gate_up_silu_tiles_norm stages.  The
 * K slice of each 64-column group that finishes last sums the group's partial
 * sums (parts->part, written as by grpo_nf4_linear_partials_attn) and applies
 * the epilogue.  group_tpart: float32 workspace of the LoRA partials per group
 * (tpart_bytes); counters: int32 workspace of counter_bytes, ZERO before the
 * first call (every call leaves it zero; calls sharing it must not overlap).
 * The hand-over to the last slice relies on a group's K slices running on one
 * XCD (linear ids equal modulo 8); each arrival checks its XCD and *xcd_err
 * becomes 1 when a group's slices ran on two XCDs (a group split over two L2s
 * leaves its counter non-zero instead): the caller checks that *xcd_err is 0
 * and the counters are zero after a run, or its outputs are not valid.
 * residual may alias h_out; row stride ld (a multiple of 4, rows 8-byte
 * aligned).  M <= 16, one LoRA segment; other shapes return GRPO_EUNSUPPORTED. */
int grpo_nf4_linear_attn_residual(const void* attn_workspace, const int32_t* context_lens,
                                  int Hq, int Hkv, int D, int block_size, int max_blocks,
                                  const uint8_t* w, const float* absmax, const float* code16,
                                  int blocksize, const void* const* lora_a,
                                  const grpo_linear_parts_t* parts, float* group_tpart,
                                  int* counters, int* xcd_err, const void* residual, void* h_out,
                                  int64_t ld, float* sumsq, grpo_stream_t stream);

/* Column groups G per row of grpo_nf4_linear_attn_residual for this shape (0 if
 * unsupported) and the bytes of its two workspaces. */
int grpo_nf4_linear_attn_residual_groups(int M, int N, int K, int r, int blocksize,
                                         size_t* tpart_bytes, size_t* counter_bytes);

/* grpo_nf4_linear_partials with x = bf16(bf16(silu(g)) * u), g and u the
 * finished gate and up halves of the gate|up projection given by its partial
 * sums (no bias or LoRA, at most 2 K slices; gate_up->N = 2 * parts->K),
 * computed while the kernel stages x: fused_silu_mul (fused_ops.py:79-112)
 * feeding down_proj in fused_mlp (fused_ops.py:184-193). */
int grpo_nf4_linear_partials_silu(const grpo_linear_parts_t* gate_up, const uint8_t* w,
                                  const float* absmax, const float* code16, int blocksize,
                                  const grpo_linear_parts_t* parts, grpo_stream_t stream);

/* act[m, j] = bf16(bf16(silu(g)) * u), g = bf16(x[m] . W[j]), u = bf16(x[m] .
 * W[I + j]) for j < I: the gate and up NF4 projections of a stacked [2I, K]
 * weight (bnb Params4bit, non-nested absmax; dequant of lora_forward.py:171-206,
 * no bias, no LoRA) with fused_silu_mul (fused_ops.py:79-112) applied, as
 * fused_mlp feeds down_proj (fused_ops.py:184-193).  act is bf16 [M, lda].
 * Fast paths only (GRPO_EUNSUPPORTED otherwise; see
 * grpo_nf4_gate_up_silu_supported); K % 256 == 0, power-of-two blocksize >= 64:
 *   M <= 16: I % 16 == 0, K <= 6144, x and the slice sums in 64 KiB of LDS;
 *     shapes with I % 8 == 0 whose 8-column units fit one workgroup per CU
 *     run those units, the others one workgroup per 16 columns;
 *   17..32 rows whose x [M, K] and unit tiles fit 160 KiB of LDS: the unit
 *     kernel on two 16-row tiles;
 *   other 17..64-row shapes with I % 8 == 0 and at most 12 units per CU: x
 *     staged in 512-column chunks, unit accumulators in registers across K;
 *   more than 64 rows (prefill chunks): the NF4 GEMM with 64 gate and the
 *     same 64 up columns per tile and SiLU*up in its epilogue (I % 8 == 0,
 *     K % 32 == 0, power-of-two blocksize >= 32). */
int grpo_nf4_gate_up_silu(const void* x, int64_t ldx, const uint8_t* w, const float* absmax,
                          const float* code16, int blocksize, int I, int K, int M, void* act,
                          int64_t lda, grpo_stream_t stream);

/* 1 if grpo_nf4_gate_up_silu takes this shape, else 0. */
int grpo_nf4_gate_up_silu_supported(int M, int I, int K, int blocksize);

/* grpo_nf4_gate_up_silu writing act (M <= 8 rows) in the fold tile layout that
 * grpo_nf4_linear_residual reads with x_tiles = 1: bf16 [ceil(I / 512) * 8][64][8]
 * (grpo_fold_tiles_elements(I) elements), element (m, k) at
 *   ((k/512 * 8 + (k/8) % 8) * 64 + m + 8 ((k/256) % 2) + 16 ((k/64) % 4)) * 8 + p(k % 8),
 *   p(e) = e/2 + 4 (e % 2),
 * so the 16-byte MFMA operands of the 64 lanes of one wave are one contiguous
 * KiB.  Slots of rows >= M and columns >= I are not written: allocate the
 * buffer zero-filled. */
int grpo_nf4_gate_up_silu_tiles(const void* x, int64_t ldx, const uint8_t* w, const float* absmax,
                                const float* code16, int blocksize, int I, int K, int M,
                                void* act_tiles, grpo_stream_t stream);

/* Elements (bf16) of a fold tile layout buffer of K columns. */
size_t grpo_fold_tiles_elements(int K);

/* grpo_nf4_gate_up_silu_tiles with x = RMSNorm(h): x[m, k] = bf16(bf16(h[m, k] *
 * inv[m]) * norm_weight[k]), inv[m] = 1 / sqrt(sum_g sumsq[m, g] / K + eps), the
 * sums as grpo_linear_finish_residual, grpo_nf4_linear_attn_residual or
 * grpo_nf4_tile_linear_residual write them (groups per row: a multiple of 4,
 * <= 256; sumsq rows and norm_weight 16-byte aligned): the
 * decoder layer's post-attention RMSNorm (fused_rmsnorm, fused_ops.py:34-77;
 * paged_kv.py:791-798) staged by the gate|up kernel.  M <= 8; shapes as
 * grpo_nf4_gate_up_silu_tiles_norm_supported. */
int grpo_nf4_gate_up_silu_tiles_norm(const void* h, int64_t ldh, const float* sumsq, int groups,
                                     const void* norm_weight, float eps, const uint8_t* w,
                                     const float* absmax, const float* code16, int blocksize,
                                     int I, int K, int M, void* act_tiles, grpo_stream_t stream);

/* 1 if grpo_nf4_gate_up_silu_tiles_norm takes this shape, else 0. */
int grpo_nf4_gate_up_silu_tiles_norm_supported(int M, int I, int K, int blocksize);

/* h_out[m, n] = bf16(residual[m, n] + bf16(x[m] . W[n])) and, for the next
 * RMSNorm, sumsq[m, g] = sum over n in [8g, 8g + 8) of h_out[m, n]^2 (float32,
 * G = N / 8 groups per row): the MLP's down_proj (NF4 weight [N, K], no bias,
 * no LoRA: fused_mlp, fused_ops.py:184-193, with the dequant of
 * lora_forward.py:171-206) followed by the decoder layer's residual add
 * (paged_kv.py:791-798) in one launch, for decode batches of M <= 8 rows.
 * x bf16 [M, ldx] (16-byte aligned, ldx % 8 == 0), or in the fold tile
 * layout when x_tiles (grpo_nf4_gate_up_silu_tiles; ldx ignored).
 * residual may be NULL (h_out = y) and may alias h_out.  Shapes: M <= 8,
 * N % 8 == 0, K % 256 == 0, K <= 16384, power-of-two blocksize >= 64
 * (grpo_nf4_linear_residual_supported); GRPO_EUNSUPPORTED otherwise. */
int grpo_nf4_linear_residual(const void* x, int64_t ldx, int x_tiles, const uint8_t* w,
                             const float* absmax, const float* code16, int blocksize, int N, int K,
                             int M, const void* residual, int64_t ldr, void* h_out, int64_t ldh,
                             float* sumsq, grpo_stream_t stream);

/* 1 if grpo_nf4_linear_residual takes this shape, else 0. */
int grpo_nf4_linear_residual_supported(int M, int N, int K, int blocksize);

/* grpo_nf4_linear_partials with x = RMSNorm(h): x[m, k] = bf16(bf16(h[m, k] *
 * inv[m]) * norm_weight[k]), inv[m] = 1 / sqrt(sum_g sumsq[m, g] / K + eps), the
 * sums of squares as grpo_nf4_linear_residual writes them (groups <= 256 per
 * row).  The decoder layer's input RMSNorm (fused_rmsnorm, fused_ops.py:34-77;
 * paged_kv.py:706-711) staged by the q|k|v projection's kernel.  h bf16 [M, ldh];
 * parts->M <= 16. */
int grpo_nf4_linear_partials_norm(const void* h, int64_t ldh, const float* sumsq, int groups,
                                  const void* norm_weight, float eps, const uint8_t* w,
                                  const float* absmax, const float* code16, int blocksize,
                                  const void* const* lora_a, const grpo_linear_parts_t* parts,
                                  grpo_stream_t stream);

/* ------------------------------------------------------- decode step --
 * Ops of the model-level decode step around the two hot-path kernels
 * (src/triton_kernels/paged_kv.py:690-820).  bf16 tensors are row-major. */

/* out[b,:] = table[ids[b],:] (table bf16 [V, H]; ids int64 [B]; ids outside
 * [0, V) give zeros).  Replaces embeddings(last_tokens) (paged_kv.py:691). */
int grpo_embedding(const int64_t* ids, const void* table, int64_t V, int H, void* out, int B,
                   grpo_stream_t stream);

/* grpo_embedding that also writes sumsq[b, t] = sum of out[b, i]^2 over
 * i = t, t + G, t + 2G, ... for t < G = grpo_embedding_sumsq_groups() (256):
 * the statistic of the first decoder layer's input RMSNorm, which the q|k|v
 * kernel stages (grpo_nf4_linear_partials_norm with groups = G). */
int grpo_embedding_sumsq(const int64_t* ids, const void* table, int64_t V, int H, void* out, int B,
                         float* sumsq, grpo_stream_t stream);

/* Groups per row written by grpo_embedding_sumsq. */
int grpo_embedding_sumsq_groups(void);

/* h = residual ? bf16(x + residual) : x  (written to h_out when residual and
 * h_out are given; h_out may alias residual); y = bf16(bf16(h * rsqrt(mean(h^2)
 * + eps)) * weight).  x, residual, h_out, y: [M, H]; weight [H].  Replaces the
 * residual add + fused_rmsnorm pair (paged_kv.py:706-711, 791-798;
 * fused_ops.py:34-77). */
int grpo_add_rmsnorm(const void* x, const void* residual, void* h_out, const void* weight,
                     void* y, int M, int H, float eps, grpo_stream_t stream);

/* h_out = bf16(residual + y) for the finished linear output y (the epilogue of
 * grpo_nf4_linear_finish: bias, LoRA), and sumsq[m, g] = sum of h_out[m, n]^2
 * over the 64 columns of group g (G = N / 64 per row, float32; N % 64 == 0): the
 * decoder layer's residual add after o_proj (paged_kv.py:791-798) with the
 * statistic of the post-attention RMSNorm, which the gate|up kernel then
 * stages (grpo_nf4_gate_up_silu_tiles_norm).  residual may be NULL and may
 * alias h_out; row stride ld for both (8-byte aligned). */
int grpo_linear_finish_residual(const grpo_linear_parts_t* parts, const void* residual,
                                void* h_out, int64_t ld, float* sumsq, grpo_stream_t stream);

/* RoPE on q and k of one token per sequence (position context_lens[b], cos/sin
 * tables bf16 [max_pos, D]), q -> q_out [B, Hq, D], rotated k and v appended to
 * the paged cache at slot context_lens[b] (same skip rules as
 * grpo_paged_kv_append).  qkv: [B, ld] rows laid out [q | k | v].  Replaces
 * fused_qkv_rope's RoPE (fused_ops.py:212-218) + repeat_kv + the KV update
 * kernel (paged_kv.py:723-752). */
int grpo_rope_append(const void* qkv, int64_t ld, int Hq, int Hkv, int D, const void* cos_table,
                     const void* sin_table, int max_pos, const int32_t* context_lens, void* q_out,
                     void* k_cache, void* v_cache, int64_t num_blocks,
                     const int32_t* block_tables, int64_t bt_stride, int block_size,
                     int max_blocks, int B, grpo_stream_t stream);

/* out[m, :N] = bf16(bf16(silu(g)) * u) with g = gate_up[m, :N], u = gate_up[m, N:2N]
 * (fused_silu_mul, fused_ops.py:79-112, 151-181). */
int grpo_silu_mul(const void* gate_up, int64_t ld, int N, void* out, int64_t ldo, int M,
                  grpo_stream_t stream);

/* Fused consumers of split-K partial sums (grpo_linear_parts_t above): each
 * first reconstructs the linear's bf16 output exactly as
 * grpo_nf4_linear_finish would, then applies its own op. */

/* grpo_add_rmsnorm with x = the finished [M, H = parts->N] linear output
 * (o_proj or down_proj). */
int grpo_add_rmsnorm_parts(const grpo_linear_parts_t* x, const void* residual, void* h_out,
                           const void* weight, void* y, float eps, grpo_stream_t stream);

/* grpo_rope_append with qkv = the finished [B = parts->M, (Hq + 2 Hkv) D]
 * q|k|v projection output. */
int grpo_qkv_rope_append_parts(const grpo_linear_parts_t* qkv, int Hq, int Hkv, int D,
                               const void* cos_table, const void* sin_table, int max_pos,
                               const int32_t* context_lens, void* q_out, void* k_cache,
                               void* v_cache, int64_t num_blocks, const int32_t* block_tables,
                               int64_t bt_stride, int block_size, int max_blocks,
                               grpo_stream_t stream);

/* grpo_silu_mul with gate_up = the finished [M, 2I] gate|up output
 * (I = parts->N / 2); out [M, I], row stride ldo. */
int grpo_silu_mul_parts(const grpo_linear_parts_t* gate_up, void* out, int64_t ldo,
                        grpo_stream_t stream);

/* Workspace bytes of grpo_lm_head_argmax (per-tile maxima) for M rows, vocab V. */
size_t grpo_lm_head_workspace_bytes(int M, int V);

/* logits[m, v] = bf16(x[m, :] . W[v, :]) (x bf16 [M, K] row stride ldx, W bf16
 * [V, K]; logits bf16 row stride ld_logits, or NULL to skip storing them) and,
 * in the workspace, the (max, first index) of every 16-column tile of every
 * row for grpo_decode_advance.  The bf16 lm_head of _step
 * (paged_kv.py:800-806) followed by the first pass of the greedy argmax
 * (paged_kv.py:444-445).  Needs V % 16 == 0, K % 256 == 0 and M <= 64; x of
 * more than 160 KiB (M * (K + 8) * 2) is staged in K chunks by a one-workgroup-
 * per-CU kernel, which takes V <= 163840 (einval otherwise). */
int grpo_lm_head_argmax(const void* x, int64_t ldx, const void* w, int V, int K, int M,
                        void* logits, int64_t ld_logits, void* workspace, size_t workspace_bytes,
                        grpo_stream_t stream);

/* grpo_lm_head_argmax with x = RMSNorm(h): x[m, k] = bf16(bf16(h[m, k] * inv[m]) *
 * norm_weight[k]), inv[m] = 1 / sqrt(sum_g sumsq[m, g] / K + eps) (groups <= 256
 * per row, as grpo_nf4_linear_residual writes them): the model's final norm
 * (paged_kv.py:806) staged by the lm_head kernel.  M <= 8. */
int grpo_lm_head_argmax_norm(const void* h, int64_t ldh, const float* sumsq, int groups,
                             const void* norm_weight, float eps, const void* w, int V, int K,
                             int M, void* logits, int64_t ld_logits, void* workspace,
                             size_t workspace_bytes, grpo_stream_t stream);

/* The lm_head weight W bf16 [V, K] rearranged for the _tiles variants below
 * (w_tiles: V * K bf16, 16-byte aligned; V % 16 == 0, K % 256 == 0): chunk
 * ((t * K / 256 + s) * 8 + j) * 64 + l of 8 bf16 holds W[16 t + l % 16][256 s +
 * 32 j + 8 (l / 16) .. + 7], the order in which one wave's loads consume a
 * vocabulary tile, so every load instruction reads 1 KiB of contiguous
 * memory.  Built once per weight (frozen during rollouts); no reference
 * counterpart (the reference reads the weight through torch/Triton). */
int grpo_lm_head_weight_tiles(const void* w, int V, int K, void* w_tiles, grpo_stream_t stream);

/* grpo_lm_head_argmax / grpo_lm_head_argmax_norm with W given in the layout of
 * grpo_lm_head_weight_tiles (same results, bit for bit).  As for the row-major
 * entries, the _norm form needs x [M, K] to fit LDS (M * (K + 8) * 2 <= 160
 * KiB; GRPO_EUNSUPPORTED otherwise); the plain form stages wider x in K
 * chunks. */
int grpo_lm_head_argmax_tiles(const void* x, int64_t ldx, const void* w_tiles, int V, int K,
                              int M, void* logits, int64_t ld_logits, void* workspace,
                              size_t workspace_bytes, grpo_stream_t stream);
int grpo_lm_head_argmax_norm_tiles(const void* h, int64_t ldh, const float* sumsq, int groups,
                                   const void* norm_weight, float eps, const void* w_tiles,
                                   int V, int K, int M, void* logits, int64_t ld_logits,
                                   void* workspace, size_t workspace_bytes,
                                   grpo_stream_t stream);

/* Greedy token of every row from grpo_lm_head_argmax's workspace (first index
 * of the maximum), written to next_tokens (may be NULL), and the decode loop's
 * per-row bookkeeping (paged_kv.py:903-980, with per-row stop lengths): for an
 * active row, generated[m, count[m]] = token (generated may be NULL), pos and
 * count advance; the row stays active while count < limit and token != eos[0];
 * tokens[m] = token; append_pos[m] = active ? pos : -1; attn_len[m] = active ?
 * pos + 1 : 0.  tokens == NULL computes next_tokens only.  active is uint8 (0/1). */
int grpo_decode_advance(const void* lm_workspace, int M, int V, int64_t* next_tokens,
                        int64_t* tokens, int32_t* pos, int32_t* count, const int32_t* limit,
                        uint8_t* active, const int64_t* eos, int64_t* generated, int64_t gen_ld,
                        int32_t* append_pos, int32_t* attn_len, grpo_stream_t stream);

/* Screened greedy lm_head: the token of grpo_lm_head_argmax[_norm] +
 * grpo_decode_advance (the first index of the largest bf16 logit, bit for
 * bit), reading an int8 copy of W to bound every logit and the bf16 tiles
 * only where the maximum can be.  No reference counterpart as a separate
 * step: the reference computes every logit (paged_kv.py:800-806) and takes the
 * argmax (:444-445); this gives the same token from fewer bytes.
 *
 * grpo_lm_head_q8_tiles: per vocabulary row v, scale[v] = max_k |W[v, k]| / 127
 * (float32), q = rint(W / scale) in [-127, 127] stored as q + 128 in wq_tiles
 * (V * K bytes, 16-byte aligned) in the order of the screening kernel's loads,
 * rnorm[v] = ||W[v, :] - scale[v] q[v, :]||_2 rounded up.  Once per weight.
 * V % 16 == 0, K % 256 == 0.  A row with a non-finite weight gets scale NaN
 * (its tiles are then always recomputed). */
int grpo_lm_head_q8_tiles(const void* w, int V, int K, void* wq_tiles, float* scale, float* rnorm,
                          grpo_stream_t stream);

/* Workspace of the screen and the exact pass: int32 arrival counters [8][32]
 * (ZERO before the first exact pass, left zero by each), the exact pass's
 * per-workgroup bests (float [8][15], int32 [8][15]), then from byte offset
 * 2048 the screen's bounds: float [M][V / 16] (per row and 16-row tile, an
 * upper bound of the tile's float32 logits), float [M][W] (per row and
 * screening workgroup, W = min(V / 16, 256), a lower bound of the largest
 * logit among its tiles) and, from the next 16-byte boundary, bf16 [V][8]
 * (per vocabulary row and row m < M, an upper bound of that logit, rounded
 * up). */
size_t grpo_lm_head_screen_workspace_bytes(int M, int V);

/* The screen: for x [M, K] (M <= 8; the _norm form stages x = RMSNorm(h) as
 * grpo_lm_head_argmax_norm does), bounds |logit - estimate| <= e from the int8
 * weight (Cauchy-Schwarz on the weight's rounding, the float16 rounding of x,
 * and the float32 summation error of both passes) and writes the bounds to the
 * workspace. */
int grpo_lm_head_screen(const void* x, int64_t ldx, const void* wq_tiles, const float* scale,
                        const float* rnorm, int V, int K, int M, void* workspace,
                        size_t workspace_bytes, grpo_stream_t stream);
int grpo_lm_head_screen_norm(const void* h, int64_t ldh, const float* sumsq, int groups,
                             const void* norm_weight, float eps, const void* wq_tiles,
                             const float* scale, const float* rnorm, int V, int K, int M,
                             void* workspace, size_t workspace_bytes, grpo_stream_t stream);

/* The exact pass after the screen (same x, M, V, K, workspace): per row, 15
 * workgroups on one XCD recompute, with grpo_lm_head_argmax_tiles' arithmetic
 * on the same operands, every 16-row tile of w_tiles
 * (grpo_lm_head_weight_tiles layout) whose upper bound reaches the row's
 * threshold (the largest lower bound, less the width of a bf16 rounding
 * interval); the last of them to arrive (an L2 counter in the workspace)
 * writes the first index of the largest bf16 logit to next_tokens.  As in
 * grpo_paged_attn_decode_qkv_merged, *xcd_err (may be NULL) becomes 1 if a
 * row's workgroups ran on two XCDs (that call's tokens are then not valid; a
 * counter is left non-zero).  The _advance_norm form stages x = RMSNorm(h) and
 * then does grpo_decode_advance's bookkeeping (next_tokens may be NULL
 * there); a row that is not active keeps its token and computes nothing.
 * workspace_bytes is checked against grpo_lm_head_screen_workspace_bytes(M, V)
 * (GRPO_EWORKSPACE below it).  Calls sharing a workspace must not overlap. */
int grpo_lm_head_exact_argmax(const void* x, int64_t ldx, const void* w_tiles, int V, int K, int M,
                              void* screen_workspace, size_t workspace_bytes, int* xcd_err,
                              int64_t* next_tokens, grpo_stream_t stream);
int grpo_lm_head_exact_advance_norm(const void* h, int64_t ldh, const float* sumsq, int groups,
                                    const void* norm_weight, float eps, const void* w_tiles, int V,
                                    int K, int M, void* screen_workspace,
                                    size_t workspace_bytes, int* xcd_err,
                                    int64_t* next_tokens, int64_t* tokens, int32_t* pos,
                                    int32_t* count, const int32_t* limit, uint8_t* active,
                                    const int64_t* eos, int64_t* generated, int64_t gen_ld,
                                    int32_t* append_pos, int32_t* attn_len, grpo_stream_t stream);

/* out[m] = first index of the maximum of logits[m, :V] (bf16, row stride ld);
 * greedy sampling of _sample_tokens / fused_logits_sampling (paged_kv.py:444-445,
 * fused_ops.py:232-234). */
int grpo_argmax_bf16(const void* logits, int64_t ld, int V, int M, int64_t* out,
                     grpo_stream_t stream);

/* Workspace bytes of grpo_sample_top_p / grpo_sample_advance for M rows: per
 * row, the counts of the row's distinct values and the draw's intermediate
 * results.  It must be zero-filled once before its first use; every call
 * leaves it zero-filled again (no memset between calls, so the calls can be
 * captured into a HIP graph).  Calls that share a workspace must be ordered
 * on one stream. */
size_t grpo_sample_workspace_bytes(int M, int V);

/* One sampled token per row from bf16 logits [M, V] (row stride ld_logits),
 * the reference's temperature / top-p rule (fused_logits_sampling,
 * fused_ops.py:236-248; _sample_tokens, paged_kv.py:437-450): scaled =
 * bf16(logits * (1 / max(T, 1e-6))); probabilities bf16(softmax(scaled)) in
 * descending order (ties by index); a token is kept while bf16(running sum) <=
 * bf16(top_p), the first always; top_p >= 1 keeps all.  The draw is the
 * inverse CDF of the kept tokens' bf16(softmax), taken in that sorted order, at
 * t = floor(draws[m] * W / 2^64), W their total in 2^-62 units.  tokens_out[m]
 * = the token, kept_out[m] (may be NULL) = the number of kept tokens.  No sort
 * and no memset.  Needs temperature > 0 (greedy decoding otherwise), V % 8 ==
 * 0, ld_logits % 8 == 0, 16-byte aligned logits and workspace. */
int grpo_sample_top_p(const void* logits, int64_t ld_logits, int M, int V, float temperature,
                      double top_p, const uint64_t* draws, int64_t* tokens_out, int32_t* kept_out,
                      void* workspace, size_t workspace_bytes, grpo_stream_t stream);

/* grpo_sample_top_p with the decode loop's bookkeeping of grpo_decode_advance
 * (paged_kv.py:800-820, :938, :978): row m's draw is SplitMix64 of (seed, m,
 * count[m]); next_tokens (may be NULL) receives the token.  Stopped rows draw
 * nothing and keep tokens[m]. */
int grpo_sample_advance(const void* logits, int64_t ld_logits, int M, int V, float temperature,
                        double top_p, uint64_t seed, int64_t* next_tokens, int64_t* tokens,
                        int32_t* pos, int32_t* count, const int32_t* limit, uint8_t* active,
                        const int64_t* eos, int64_t* generated, int64_t gen_ld,
                        int32_t* append_pos, int32_t* attn_len, void* workspace,
                        size_t workspace_bytes, grpo_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* GRPO_HIP_H */
