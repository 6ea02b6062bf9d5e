/*
 * slmturbo.h -- C ABI of libslmturbo_hip.so, the MI355X (gfx950) implementation
 * of slm-turbo's fused 4-bit KV-cache dequant + decode-attention path.
 *
 * Every entry point takes plain device pointers, sizes and strides (in
 * elements), launches asynchronously on the given HIP stream and returns a
 * status code; 0 means the work was enqueued.  On failure nothing is launched
 * and slmt_last_error() returns a message for the calling thread, worded like
 * the reference's TORCH_CHECK messages.  No entry point allocates device
 * memory: outputs and workspaces are owned by the caller.
 *
 * Data formats (unchanged from the reference, so caches written by either side
 * are interchangeable):
 *   - fp16 is IEEE binary16, passed as raw 16-bit storage;
 *   - a packed byte holds dim 2j in its low nibble and dim 2j+1 in its high
 *     nibble (reference kernels/kv_dequant_kernels.cuh:14-17);
 *   - paged cache: uint8 [num_blocks, block_size, KV, D+8]; each slot holds
 *     D/2 bytes of K codes, D/2 bytes of V codes, then fp16 k_min, k_step,
 *     v_min, v_step (reference kernels/kv_dequant_kernels.cuh:511-518,666-670;
 *     adapters/vllm_adapter.py:300-308).
 * Supported head_dim D: 64, 80, 128 (reference kernels/kv_dequant.py:113).
 * The softmax scale is 1/sqrt(D) (reference kernels/kv_dequant_kernels.cuh:167).
 */
#ifndef SLMTURBO_H
#define SLMTURBO_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* slmt_stream_t;  /* a hipStream_t; NULL = the null stream */

enum {
  SLMT_OK = 0,
  SLMT_ERR_INVALID = 1,      /* argument validation failed */
  SLMT_ERR_UNSUPPORTED = 2,  /* valid request outside what this build supports */
  SLMT_ERR_HIP = 3           /* a HIP runtime call or launch failed */
};

enum { SLMT_OUT_F32 = 0, SLMT_OUT_F16 = 1 };

/* Message for the last failing call on this thread ("" if none). */
const char* slmt_last_error(void);

/* ABI version of this library (SLMT_ABI_VERSION). */
#define SLMT_ABI_VERSION 3
int slmt_abi_version(void);

/* Bytes of caller-owned workspace the attention entry points need.  A
 * workspace starts with a fixed region of 2^20 arrival counters (one per
 * (sequence, head group) pair of a call) followed by split-sequence partial
 * results.  It must be zero-filled once after allocation; every call leaves
 * its counters at zero again, so one workspace can be reused by calls of any
 * shape that are ordered on one stream (calls that overlap must not share
 * one).  num_seqs is the batch size B (for prefill: the number of query rows
 * M).  Returns -1 and sets the error on invalid sizes. */
int64_t slmt_attention_workspace_bytes(int num_seqs, int num_heads, int num_kv_heads,
                                       int head_dim);

/*
 * Quantize-on-write store.  Replaces kv_quantize_store_cuda
 * (reference kernels/kv_dequant_cuda.cu:415-456, kernel
 * kernels/kv_dequant_kernels.cuh:816-919), bound from kernels/kv_dequant.py:220-233.
 *   key, value:   fp16 [N, KV, D]; row (token, head) at base + t*token_stride + h*D
 *   kv_cache:     uint8 [num_blocks, block_size, KV, D+8], contiguous
 *   slot_mapping: int64 [N]; slot = block * block_size + pos; slot < 0 is skipped,
 *                 slot >= num_blocks*block_size is skipped as out of range
 * Per (token, kv head): fp32 min/max, step = (max-min)/15 (1 when !(step>0)),
 * code = clamp((int)((x-min)/step + 0.5f), 0, 15); packs K, V and the fp16 rulers.
 * Bit-exact with the reference store.
 */
int slmt_quantize_store(const void* key, int64_t key_token_stride,
                        const void* value, int64_t value_token_stride,
                        void* kv_cache, int64_t num_blocks, int block_size,
                        const int64_t* slot_mapping, int64_t num_tokens,
                        int num_kv_heads, int head_dim, slmt_stream_t stream);

/*
 * Per-channel asymmetric 4-bit quantizer of the standalone path (host torch
 * code in the reference: kernels/benchmark/benchmark.py:26-56), on the GPU.
 *   x:      fp16 [KV, S, D] contiguous
 *   packed: uint8 [KV, S, D/2] out;  scale, zero: fp16 [KV, D] out
 * Every arithmetic step rounds to fp16 like the reference's torch ops;
 * bit-exact with kernels/benchmark/benchmark.py:26-56.
 */
int slmt_quantize_per_channel(const void* x, int num_kv_heads, int seq_len, int head_dim,
                              void* packed, void* scale, void* zero, slmt_stream_t stream);

/*
 * Per-channel append with fixed rulers: the reference's quantize_tensor(x,
 * scale, zero_point) (host torch code, kernels/benchmark/benchmark.py:45-56),
 * which its model harness uses to pack new tokens with the rulers frozen at
 * the first decode (:213-216), on the GPU.
 *   x:      fp16, element (h, s, d) at x + h*x_head_stride + s*x_seq_stride + d
 *           (strides in elements, even; x 4-byte aligned)
 *   scale, zero: fp16 [KV, D] contiguous, 4-byte aligned
 *   packed: uint8, byte (h, s, j) at packed + h*out_head_stride + s*out_seq_stride + j
 *           (j < D/2; e.g. a slice of a preallocated [KV, capacity, D/2] cache)
 * q = clamp(round(x / scale) + zero, 0, 15) with an fp16 result after each op,
 * bit-exact with the reference's torch arithmetic; dim 2j in the low nibble.
 */
int slmt_quantize_with_rulers(const void* x, int64_t x_head_stride, int64_t x_seq_stride, int num_kv_heads,
                              int seq_len, int head_dim, const void* scale, const void* zero, void* packed,
                              int64_t out_head_stride, int64_t out_seq_stride, slmt_stream_t stream);

/*
 * Batched paged decode over the packed per-token cache: one launch for the
 * whole batch.  Extends kv_dequant_decode_per_token_paged_attention_cuda
 * (reference kernels/kv_dequant_cuda.cu:355-410, kernel
 * kernels/kv_dequant_kernels.cuh:671-801), which the reference's vLLM
 * backend calls once per request (adapters/vllm_adapter.py:271-279).
 *   q:            fp16, element (b, h, d) at q + b*q_seq_stride + h*q_head_stride + d
 *   kv_cache:     uint8 [num_blocks, block_size, KV, D+8]
 *   block_tables: int32 or int64 (block_table_bits = 32|64); row b at
 *                 block_tables + b*block_table_stride, >= ceil(L_b/block_size) entries
 *   seq_lens:     int32 [B] on the device, or NULL to use fixed_seq_len for every b
 *   out:          fp32 or fp16 (out_dtype), element (b, h, d) at
 *                 out + b*out_seq_stride + h*out_head_stride + d
 * GQA: query head h reads kv head h / (H / num_kv_heads).  Sequences of
 * length 0 produce zeros.
 * workspace: slmt_attention_workspace_bytes(B, num_heads, num_kv_heads, D).
 */
int slmt_decode_paged_batched(const void* q, int64_t q_seq_stride, int64_t q_head_stride,
                              const void* kv_cache, int64_t num_blocks, int block_size,
                              const void* block_tables, int block_table_bits,
                              int64_t block_table_stride,
                              const int32_t* seq_lens, int fixed_seq_len,
                              int num_seqs, int num_heads, int num_kv_heads, int head_dim,
                              void* out, int out_dtype, int64_t out_seq_stride,
                              int64_t out_head_stride, void* workspace, int64_t workspace_bytes,
                              slmt_stream_t stream);

/*
 * Allocation-free batched paged decode.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory or pass a workspace (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Arguments, kernels and results are those of
 * slmt_decode_paged_batched without the workspace: the library keeps one
 * static device scratch array of SLMT_NOALLOC_SCRATCH_BYTES per GPU for the
 * life of the process, and calls whose workspace
 * (slmt_attention_workspace_bytes) would exceed it fail with
 * SLMT_ERR_UNSUPPORTED.  All calls on one GPU share that array: calls must be
 * ordered (one stream, or synchronized); overlapping calls race.  Nothing in
 * the call allocates.
 */
#define SLMT_NOALLOC_SCRATCH_BYTES (16 * 1024 * 1024)
int slmt_decode_paged_batched_noalloc(const void* q, int64_t q_seq_stride, int64_t q_head_stride,
                                      const void* kv_cache, int64_t num_blocks, int block_size,
                                      const void* block_tables, int block_table_bits,
                                      int64_t block_table_stride, const int32_t* seq_lens,
                                      int fixed_seq_len, int num_seqs, int num_heads,
                                      int num_kv_heads, int head_dim, void* out, int out_dtype,
                                      int64_t out_seq_stride, int64_t out_head_stride,
                                      slmt_stream_t stream);

/*
 * Paged decode of ONE request.  Replaces
 * kv_dequant_decode_per_token_paged_attention_cuda (reference
 * kernels/kv_dequant_cuda.cu:355-410), bound from kernels/kv_dequant.py:236-257.
 *   q:           fp16 [H, 1, D] contiguous
 *   kv_cache:    uint8 [num_blocks, block_size, KV, D+8]
 *   block_table: int64 [>= ceil(seq_len/block_size)] on the device
 *   out:         fp32 [H, 1, D]
 * seq_len 0 writes zeros (the Python binding returns NaN like the reference's
 * 0/0 softmax).  A batch of one through slmt_decode_paged_batched.
 * workspace: slmt_attention_workspace_bytes(1, num_heads, num_kv_heads, D).
 */
int slmt_decode_paged(const void* q, const void* kv_cache, int64_t num_blocks, int block_size,
                      const int64_t* block_table, int seq_len, int num_heads, int num_kv_heads,
                      int head_dim, float* out, void* workspace, int64_t workspace_bytes,
                      slmt_stream_t stream);

/*
 * Per-token decode over contiguous buffers.  Replaces
 * kv_dequant_decode_per_token_attention_cuda (reference
 * kernels/kv_dequant_cuda.cu:277-350, kernel kernels/kv_dequant_kernels.cuh:528-655).
 *   q: fp16 [H, 1, D]; k_packed, v_packed: uint8 [KV_t, S, D/2];
 *   k_min, k_step, v_min, v_step: fp16 [KV_t, S]; out: fp32 [H, 1, D].
 * GQA map uses num_kv_heads (<= KV_t); block_n (32|64) is accepted for API
 * parity and does not change the result beyond rounding.
 */
int slmt_decode_per_token(const void* q, const void* k_packed, const void* k_min,
                          const void* k_step, const void* v_packed, const void* v_min,
                          const void* v_step, int num_heads, int kv_tensor_heads,
                          int num_kv_heads, int seq_len, int head_dim, int block_n,
                          float* out, void* workspace, int64_t workspace_bytes,
                          slmt_stream_t stream);

/*
 * Per-channel decode.  Replaces kv_dequant_decode_attention_cuda (reference
 * kernels/kv_dequant_cuda.cu:83-177, kernel kernels/kv_dequant_kernels.cuh:113-275).
 *   k_scale, k_zero, v_scale, v_zero: fp16 [KV_t, D]; use_quant = 0 attends
 *   over the raw nibble values.  Other arguments as slmt_decode_per_token.
 */
int slmt_decode_per_channel(const void* q, const void* k_packed, const void* k_scale,
                            const void* k_zero, const void* v_packed, const void* v_scale,
                            const void* v_zero, int num_heads, int kv_tensor_heads,
                            int num_kv_heads, int seq_len, int head_dim, int block_n,
                            int use_quant, float* out, void* workspace,
                            int64_t workspace_bytes, slmt_stream_t stream);

/*
 * Per-channel prefill.  Replaces kv_dequant_prefill_attention_cuda (reference
 * kernels/kv_dequant_cuda.cu:182-272, kernel kernels/kv_dequant_kernels.cuh:293-502).
 *   q: fp16 [H, M, D]; out: fp32 [H, M, D]; causal masks key n > query m
 *   (both indexed from 0).  block_m/block_n are validated like the reference
 *   (16|32, 32|64, (16,32) only for D != 64) and do not change the result.
 *   workspace: slmt_attention_workspace_bytes(M, H, num_kv_heads, D); head_dim
 *   64 and 128 run on the matrix cores and use none of it (it may be NULL
 *   there), head_dim 80 needs it.
 */
int slmt_prefill_per_channel(const void* q, const void* k_packed, const void* k_scale,
                             const void* k_zero, const void* v_packed, const void* v_scale,
                             const void* v_zero, int num_heads, int kv_tensor_heads,
                             int num_kv_heads, int num_queries, int seq_len, int head_dim,
                             int block_m, int block_n, int causal, int use_quant,
                             float* out, void* workspace, int64_t workspace_bytes,
                             slmt_stream_t stream);

/*
 * Measurement hook; it has no counterpart in the reference and is for
 * benchmark harnesses (bench.py).  slmt_kernel_timing(1) makes each following
 * batched paged decode call that runs a whole-row kernel time that kernel
 * alone (not the merge of split sequences that follows it) with a HIP event
 * pair stamped from the kernel's own dispatch (hipExtLaunchKernelGGL), for up
 * to 4096 calls; slmt_kernel_timing(0) stops.  The events are created when
 * timing is first switched on (on the device current then), so a timed call
 * creates nothing.  slmt_kernel_timing_read waits for the recorded events,
 * writes up to max_n durations in microseconds (call order) to us, forgets
 * all recorded pairs and returns how many it wrote, or -1 on a HIP error.
 * slmt_kernel_timing_kernel names the kernel of the most recent timed call
 * (instantiation and unit, e.g. "mfma_kernel<128,8,1> (matrix cores)"; ""
 * before any), a string owned by the library.
 */
int slmt_kernel_timing(int enable);
int slmt_kernel_timing_read(float* us, int max_n);
const char* slmt_kernel_timing_kernel(void);

#ifdef __cplusplus
}
#endif

#endif /* SLMTURBO_H */
