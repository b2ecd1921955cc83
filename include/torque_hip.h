/*
 * torque_hip.h -- C ABI of the MI355X (gfx950) packed rotated KV-cache decode path.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t.
 * The library allocates no device memory; the caller owns all buffers
 * (slabs, centroids, signs, workspaces, outputs).  Its only device state is
 * the fixed per-GPU scratch array of tq_decode_noalloc, the entry point for
 * callers that cannot allocate a workspace.  Its only other state is one pair
 * of HIP events per device, created on the first timed call there that passes
 * no merge events of its own (tq_decode_timed, tq_decode_scaled_timed,
 * tq_decode_dense_timed) and shared by every stream.  Kernels are
 * launched asynchronously on `stream`.  Return value: TQ_OK (0) or a negative
 * TQ_ERR_* code; tq_last_error() gives the message (thread-local).
 *
 * Layouts (row-major, contiguous):
 *   packed code slab  uint32 [L, Hkv, capacity, W],  W = ceil(D * bits / 32)
 *                     (reference docs/contracts/packed-kv-layout.md:5-24)
 *   queries           [L, Hq, D]   (float32 or float16)
 *   outputs           float32 [L, Hq, D]
 *   query head qh reads KV head qh / (Hq / Hkv)  (reference cache_mlx.py:706-722)
 *
 * Citations below name the reference interface each entry point replaces
 * (paths relative to src/torque_mlx/ of cbun/torque-mlx).
 */
#ifndef TORQUE_HIP_H
#define TORQUE_HIP_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TQ_ABI_VERSION 4

enum {
  TQ_OK = 0,
  TQ_ERR_BAD_ARG = -1,     /* shape / pointer / range error (Python: ValueError) */
  TQ_ERR_UNSUPPORTED = -2, /* bits or head_dim outside {2,3,4} x {64,128,256} (ValueError) */
  TQ_ERR_LAUNCH = -3       /* HIP launch failure (Python: RuntimeError) */
};

enum { TQ_F32 = 0, TQ_F16 = 1 };

/* tq_append / tq_quantize_dequantize flags (reference cache_mlx.py:52-54) */
enum { TQ_ROTATE_KEYS = 1, TQ_ROTATE_VALUES = 2 };
/* tq_decode / tq_decode_dense flags (reference cache_mlx.py:188-196, 225-232).
 * The split kernel (no reference counterpart): the float16-split matrix
 * kernel can run for groups of 4 query heads with 4-bit rows at head_dim
 * 64 / 128 / 256 or 2-bit rows at head_dim 128, and by default does where
 * its split plan gives every split at least 4 blocks of 128 rows (8 at
 * head_dim 256); elsewhere the float32 split kernel runs.  Both accumulate in float32.  TQ_F32_PRODUCTS selects
 * the float32 kernel, TQ_MATRIX_PRODUCTS the matrix kernel wherever it can
 * run (the two exclude each other: TQ_ERR_BAD_ARG).  tq_decode_scaled always
 * runs the float32 split kernel.
 *
 * Reproducibility: both split kernels deal their work statically and the
 * merge sums the splits in a fixed order, so a decode returns bit-identical
 * outputs on every call, on any stream and in every graph replay, as the
 * reference's decode does (cache.py:98-140, mlx_ops.py:571-595). */
enum { TQ_ROTATE_QUERY = 1, TQ_INVERSE_OUTPUT = 2, TQ_F32_PRODUCTS = 4, TQ_MATRIX_PRODUCTS = 8 };

int tq_abi_version(void);
const char* tq_last_error(void);

/* Structured Hadamard rotation of `rows` vectors of length head_dim.
 * inverse == 0: y = sL * (H (sR * x)) / sqrt(D)   (rotation.py:88-94, 113-123)
 * inverse != 0: y = sR * (H (sL * x)) / sqrt(D)   (rotation.py:96-102, 126-136)
 * Bit-identical to the reference's float32 numpy transform (rotation.py:19-32). */
int tq_fwht(const void* x, int x_dtype, float* y, int64_t rows, int head_dim, const float* signs_left,
            const float* signs_right, int inverse, hipStream_t stream);

/* Quantize already-rotated float32 rows by boundary count and bit-pack them:
 * values [rows, D] -> packed [rows, W].  Replaces quantize_and_pack_rows_metal
 * (mlx_ops.py:256-292, 342-371); bit-exact to quantize + pack_indices_batched
 * (quantization.py:139-148, 176-201). */
int tq_quantize_pack(const float* values, int64_t rows, int head_dim, int bits, const float* boundaries,
                     uint32_t* packed, hipStream_t stream);

/* Fused rotate -> quantize -> bit-pack append of seq_new tokens for every
 * layer and KV head, written in place at slab position `offset`.
 * keys/values [L, Hkv, seq_new, D] (dtype TQ_F32 or TQ_F16).  Flags select
 * which streams are rotated.  Replaces TorqueKVCacheMLX._append_packed_tokens
 * and quantize_and_pack_rows_dual_metal (cache_mlx.py:396-418, 504-521;
 * mlx_ops.py:295-339, 374-412). */
int tq_append(const void* keys, const void* values, int dtype, int num_layers, int kv_heads, int64_t seq_new,
              int head_dim, int bits, const float* signs_left, const float* signs_right, int flags,
              const float* key_boundaries, const float* value_boundaries, uint32_t* key_codes,
              uint32_t* value_codes, int64_t capacity, int64_t offset, hipStream_t stream);

/* Per-vector scales (opt-in extension; the reference has none -- its codes
 * index one global codebook per stream, quantization.py:120-148).  The
 * rotated row x is quantized as x / s with s = sqrt(mean(x^2)) (1 for a zero
 * row), one float32 s per (layer, KV head, token) and stream, stored in scale
 * slabs [L, Hkv, capacity] beside the code slabs.  The codes equal the
 * reference packer applied to x / s; the dequantized token is centroid x s.
 * Same arguments as tq_append plus the two scale slabs. */
int tq_append_scaled(const void* keys, const void* values, int dtype, int num_layers, int kv_heads, int64_t seq_new,
                     int head_dim, int bits, const float* signs_left, const float* signs_right, int flags,
                     const float* key_boundaries, const float* value_boundaries, uint32_t* key_codes,
                     uint32_t* value_codes, float* key_scales, float* value_scales, int64_t capacity,
                     int64_t offset, hipStream_t stream);

/* Rotate (per flags) -> quantize -> dequantize to dense float32 centroid values,
 * rows [rows, D] -> out [rows, D]; values/value_out may be NULL.  Replaces
 * TorqueKVCacheMLX._quantize_rows on the current token (cache_mlx.py:246-255, 496-502). */
int tq_quantize_dequantize(const void* keys, const void* values, int dtype, int64_t rows, int head_dim, int bits,
                           const float* signs_left, const float* signs_right, int flags,
                           const float* key_boundaries, const float* value_boundaries,
                           const float* key_centroids, const float* value_centroids, float* key_out,
                           float* value_out, hipStream_t stream);

/* tq_quantize_dequantize with per-vector scales (see tq_append_scaled):
 * out = centroid(code(x / s)) x s.  The current token of a scaled cache. */
int tq_quantize_dequantize_scaled(const void* keys, const void* values, int dtype, int64_t rows, int head_dim,
                                  int bits, const float* signs_left, const float* signs_right, int flags,
                                  const float* key_boundaries, const float* value_boundaries,
                                  const float* key_centroids, const float* value_centroids, float* key_out,
                                  float* value_out, hipStream_t stream);

/* Unpack + dequantize the first seq_len tokens of `groups` slab rows:
 * codes [groups, capacity, W] -> out float32 [groups, seq_len, D].
 * Replaces TorqueKVCache.export_dequantized (cache.py:189-214). */
int tq_unpack_dequantize(const uint32_t* codes, int64_t groups, int64_t capacity, int64_t seq_len, int head_dim,
                         int bits, const float* centroids, float* out, hipStream_t stream);

/* tq_unpack_dequantize of a scaled slab: out = centroid x scale, scales
 * [groups, capacity] float32 (see tq_append_scaled). */
int tq_unpack_dequantize_scaled(const uint32_t* codes, const float* scales, int64_t groups, int64_t capacity,
                                int64_t seq_len, int head_dim, int bits, const float* centroids, float* out,
                                hipStream_t stream);

/* Split count a decode call over `bits`-bit rows (0 for dense rows) with
 * decode `flags` uses when n_splits <= 0 is passed, on num_cus compute units
 * (<= 0: the current device's).  The sequence is dealt out to the splits in
 * blocks of one workgroup iteration (split s takes blocks s, s + n, s + 2n,
 * ...); an explicit n_splits above the number of blocks is lowered to it. */
int tq_decode_default_splits(int num_layers, int kv_heads, int query_heads, int head_dim, int bits, int flags,
                             int64_t seq_len, int num_cus);

/* Name of the split kernel a tq_decode call over `bits`-bit packed rows with
 * decode `flags`, a query of `query_dtype`, seq_len tokens and n_splits
 * (<= 0: the default) launches on num_cus compute units (<= 0: the current
 * device's): "decode_mx_kernel<D,QF16>" (the float16-split matrix kernel;
 * "decode_mx_kernel<D,QF16,2>" for 2-bit rows) or
 * "decode_kernel<PackedB<bits>,D,<heads per group>>" (the float32 kernel;
 * tq_decode_scaled always runs this one).  For profiles and benchmarks; no
 * reference counterpart.  NULL on bad arguments (tq_last_error). */
const char* tq_decode_split_kernel(int num_layers, int kv_heads, int query_heads, int head_dim, int bits, int flags,
                                   int query_dtype, int64_t seq_len, int n_splits, int num_cus);

/* Bytes of workspace tq_decode / tq_decode_dense need for n_splits splits
 * (n_splits <= 0: enough for the default split count on any sequence length
 * with num_cus compute units).  The workspace holds per-split partial results
 * between the two launches of one call; it needs no initialisation.  Calls
 * that share one workspace must be ordered (same stream).  Every decode entry
 * point takes the workspace's size in bytes (workspace_bytes) and returns
 * TQ_ERR_BAD_ARG, before any launch, when it is smaller than the split plan
 * the call resolves to needs. */
size_t tq_decode_workspace_bytes(int num_layers, int kv_heads, int query_heads, int head_dim, int n_splits,
                                 int num_cus);

/* Fused packed-code decode attention for one query token per query head:
 * optional query rotation, split-K over the sequence with an online softmax
 * in the rotated basis, log-sum-exp merge of the splits and optional inverse
 * rotation.  One launch when the sequence is not split (n_splits resolves to
 * 1), otherwise the split kernel followed by a small merge kernel.  current_keys / current_values
 * (float32 [L, Hkv, D], already rotated and dequantized, or NULL) join the
 * softmax as one extra dense token.  Replaces decode_packed_attention_split_batched
 * (mlx_ops.py:571-595), ..._with_current (mlx_ops.py:598-660),
 * decode_packed_attention (mlx_ops.py:663-692) and the decode flow of
 * TorqueKVCacheMLX.decode_mlx / decode_mlx_with_current (cache_mlx.py:173-302). */
int tq_decode(const void* query, int query_dtype, int num_layers, int query_heads, int kv_heads, int head_dim,
              int bits, const uint32_t* key_codes, const uint32_t* value_codes, int64_t capacity,
              int64_t seq_len, const float* key_centroids, const float* value_centroids,
              const float* signs_left, const float* signs_right, int flags, const float* current_keys,
              const float* current_values, int n_splits, void* workspace, size_t workspace_bytes, float* out,
              hipStream_t stream);

/* tq_decode without a caller workspace and without allocating: the split-K
 * partials go to a static scratch array of 8 MiB held by the library on each
 * GPU (device memory, kept until the process ends; its address is looked up
 * once per device on the first call there).  No counterpart in the reference:
 * it is for callers that cannot allocate -- code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc -- and calls no
 * hipMalloc, hipFree or other allocating routine.  Same arguments and results
 * as tq_decode minus the workspace.  A call whose resolved split plan needs
 * more than 8 MiB (tq_decode_workspace_bytes) returns TQ_ERR_BAD_ARG before
 * any launch; pass fewer splits or fewer layers.  Every call on one GPU shares
 * that GPU's scratch: calls that overlap on one GPU (different streams, or
 * threads without ordering) race and must not be issued.  The first call on a
 * device must be made outside stream capture (it looks the scratch address
 * up); made inside one, it returns TQ_ERR_BAD_ARG before enqueueing anything. */
int tq_decode_noalloc(const void* query, int query_dtype, int num_layers, int query_heads, int kv_heads,
                      int head_dim, int bits, const uint32_t* key_codes, const uint32_t* value_codes,
                      int64_t capacity, int64_t seq_len, const float* key_centroids, const float* value_centroids,
                      const float* signs_left, const float* signs_right, int flags, const float* current_keys,
                      const float* current_values, int n_splits, float* out, hipStream_t stream);

/* tq_decode over slabs written by tq_append_scaled: a token's score is
 * multiplied by its key scale and its value by its value scale (scales
 * [L, Hkv, capacity] float32).  current_keys / current_values, when given,
 * are already scaled (tq_quantize_dequantize_scaled).  No counterpart in the
 * reference, which has no per-vector scales. */
int tq_decode_scaled(const void* query, int query_dtype, int num_layers, int query_heads, int kv_heads, int head_dim,
                     int bits, const uint32_t* key_codes, const uint32_t* value_codes, const float* key_scales,
                     const float* value_scales, int64_t capacity, int64_t seq_len, const float* key_centroids,
                     const float* value_centroids, const float* signs_left, const float* signs_right, int flags,
                     const float* current_keys, const float* current_values, int n_splits, void* workspace,
                     size_t workspace_bytes, float* out, hipStream_t stream);

/* tq_decode_scaled with HIP events bound to the split kernel's launch
 * (start/stop may be NULL), as tq_decode_timed. */
int tq_decode_scaled_timed(const void* query, int query_dtype, int num_layers, int query_heads, int kv_heads,
                           int head_dim, int bits, const uint32_t* key_codes, const uint32_t* value_codes,
                           const float* key_scales, const float* value_scales, int64_t capacity, int64_t seq_len,
                           const float* key_centroids, const float* value_centroids, const float* signs_left,
                           const float* signs_right, int flags, const float* current_keys,
                           const float* current_values, int n_splits, void* workspace, size_t workspace_bytes,
                           float* out, hipStream_t stream, hipEvent_t start, hipEvent_t stop);

/* Append one token to the packed slabs and decode with it in one launch:
 * the same as tq_append(new token at row seq_len) followed by
 * tq_decode(seq_len + 1) -- the packed words are identical and the output
 * matches to float rounding -- but the new token's codes are produced inside
 * the decode's split-0 workgroups and the token joins the softmax from
 * registers, saving the append launch of every decode step.  new_keys /
 * new_values are [L, Hkv, D] in kv_dtype (TQ_F32 or TQ_F16, independent of
 * the query's query_dtype; the token is quantized from its own values, as
 * the reference quantizes float32 K/V, cache_mlx.py:442-466); append_flags
 * TQ_ROTATE_KEYS / TQ_ROTATE_VALUES as for tq_append, decode_flags as for
 * tq_decode.  seq_len (tokens already in the slabs) must be below capacity.
 * Replaces the per-layer decode_mlx_with_current + append pair of the
 * reference's Qwen decode step (qwen_mlx.py:826-828; cache_mlx.py:236-302,
 * 151-171). */
int tq_decode_append(const void* query, int query_dtype, const void* new_keys, const void* new_values, int kv_dtype,
                     int num_layers, int query_heads, int kv_heads, int head_dim, int bits, uint32_t* key_codes,
                     uint32_t* value_codes, int64_t capacity, int64_t seq_len, const float* key_centroids,
                     const float* value_centroids, const float* key_boundaries, const float* value_boundaries,
                     const float* signs_left, const float* signs_right, int append_flags, int decode_flags,
                     int n_splits, void* workspace, size_t workspace_bytes, float* out, hipStream_t stream);

/* Same as tq_decode; start/stop events (may be NULL) are bound to the split
 * kernel itself, so hipEventElapsedTime gives its execution time (the merge
 * kernel, when launched, follows it on the stream).  When either event is
 * given, the merge launch is profiled as well, with a pair of events the
 * library owns (one pair per device, shared by every stream of that device and
 * never read): a dispatch with profiling that follows one without starts late
 * on most of the GPU's XCDs, and the split kernel's events would count that
 * delay as its own time.  tq_decode_step_timed takes the merge's events from
 * the caller instead. */
int tq_decode_timed(const void* query, int query_dtype, int num_layers, int query_heads, int kv_heads,
                    int head_dim, int bits, const uint32_t* key_codes, const uint32_t* value_codes,
                    int64_t capacity, int64_t seq_len, const float* key_centroids, const float* value_centroids,
                    const float* signs_left, const float* signs_right, int flags, const float* current_keys,
                    const float* current_values, int n_splits, void* workspace, size_t workspace_bytes, float* out,
                    hipStream_t stream, hipEvent_t start, hipEvent_t stop);

/* tq_decode with caller-owned HIP events bound to each of its launches:
 * split_start / split_stop to the split kernel, merge_start / merge_stop to
 * the merge kernel (both NULL: the library's pair, as in tq_decode_timed;
 * one NULL: TQ_ERR_BAD_ARG).  A call that resolves to one split launches no
 * merge kernel and records neither merge event.  The time of one decode step
 * is the sum of the two kernels' elapsed times.  For benchmarks; no reference
 * counterpart. */
int tq_decode_step_timed(const void* query, int query_dtype, int num_layers, int query_heads, int kv_heads,
                         int head_dim, int bits, const uint32_t* key_codes, const uint32_t* value_codes,
                         int64_t capacity, int64_t seq_len, const float* key_centroids, const float* value_centroids,
                         const float* signs_left, const float* signs_right, int flags, const float* current_keys,
                         const float* current_values, int n_splits, void* workspace, size_t workspace_bytes,
                         float* out, hipStream_t stream, hipEvent_t split_start, hipEvent_t split_stop,
                         hipEvent_t merge_start, hipEvent_t merge_stop);

/* Dense-KV decode attention with the same split-K structure, for float16 or
 * float32 K/V slabs [L, Hkv, capacity, D].  With kv_dtype TQ_F16 this is the
 * fp16-dense comparator of the reference's qwen-decode benchmark (MLX-LM
 * KVCache + scaled_dot_product_attention, qwen_benchmark.py:313-314, 395-402);
 * with TQ_F32 and the rotation flags it is the fp32 rotated baseline of the
 * synthetic benchmark (benchmarking.py:62-71). */
int tq_decode_dense(const void* query, int query_dtype, const void* keys, const void* values, int kv_dtype,
                    int num_layers, int query_heads, int kv_heads, int head_dim, int64_t capacity, int64_t seq_len,
                    const float* signs_left, const float* signs_right, int flags, int n_splits, void* workspace,
                    size_t workspace_bytes, float* out, hipStream_t stream);

int tq_decode_dense_timed(const void* query, int query_dtype, const void* keys, const void* values,
                          int kv_dtype, int num_layers, int query_heads, int kv_heads, int head_dim,
                          int64_t capacity, int64_t seq_len, const float* signs_left, const float* signs_right,
                          int flags, int n_splits, void* workspace, size_t workspace_bytes, float* out,
                          hipStream_t stream, hipEvent_t start, hipEvent_t stop);

/* Raw (unscaled) packed scores: query [B, D] (rotated), codes [B, S, W] -> scores [B, S].
 * Replaces score_packed_query_batched (mlx_ops.py:113-145, 501-531). */
int tq_score_packed(const float* query, const uint32_t* codes, int batch, int64_t seq_len, int head_dim, int bits,
                    const float* centroids, float* scores, hipStream_t stream);

/* Row softmax of scale * scores: [B, S] -> [B, S] (the mx.softmax of mlx_ops.py:588). */
int tq_softmax_rows(const float* scores, int batch, int64_t seq_len, float scale, float* weights,
                    hipStream_t stream);

/* Weighted packed value sum: weights [B, S], codes [B, S, W] -> out [B, D].
 * Replaces accumulate_packed_values_batched (mlx_ops.py:148-178, 534-568). */
int tq_accumulate_packed(const float* weights, const uint32_t* codes, int batch, int64_t seq_len, int head_dim,
                         int bits, const float* centroids, float* out, hipStream_t stream);

/* Measurement helper, no counterpart in the reference: streams `bytes` bytes
 * (a multiple of 16, 16-byte aligned) through nontemporal 16-byte loads,
 * four in flight per thread, over n_blocks workgroups of 512 threads (<= 0:
 * one per compute unit) -- the device's streaming-read
 * ceiling that the decode kernels' bandwidth is compared with.  `sink` holds
 * n_blocks floats and is written only in the (practically impossible) case
 * that the xor of the data equals a fixed pattern.  start/stop events (may be
 * NULL) are bound to the kernel as in tq_decode_timed. */
int tq_stream_read(const void* data, size_t bytes, float* sink, int n_blocks, hipStream_t stream, hipEvent_t start,
                   hipEvent_t stop);

#ifdef __cplusplus
}
#endif

#endif /* TORQUE_HIP_H */
