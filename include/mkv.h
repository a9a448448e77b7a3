/*
 * mkv.h — C ABI of the MI355X (gfx950) KV-cache hot path.
 *
 * The library behind this header (libmkv.so) implements the paged-KV
 * operators of the mini-kvllm engine (src/myvllm/layers/attention.py in the
 * reference) as hand-written HIP kernels:
 *
 *   K1  slot-mapped KV append: plain copy, or fused per-tensor FP8 /
 *       per-token-head FP8 / per-token-head INT8 quantisation
 *   K2  paged decode attention (GQA-shared K/V tiles; stream-K or split-K,
 *       partials merged by log-sum-exp)
 *   K3  paged / contiguous causal prefill attention on MFMA
 *   K4  block-table gather (shared device functions + a standalone kernel)
 *
 * Conventions
 *   - Every pointer is a device pointer unless stated otherwise.  The library
 *     never allocates, frees or synchronises; callers own all memory.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *     Work is only enqueued; no host reads of device data happen inside.
 *   - Every function returns an int status: 0 = ok, negative = argument or
 *     unsupported-combination error (see MKV_ERR_*), positive = a hipError_t
 *     reported by the launch.  mkv_status_string() names each code.
 *   - Element counts and strides are in elements of the tensor's dtype.
 *   - KV pool layout per layer: (num_blocks, block_size, num_kv_heads,
 *     head_dim), contiguous; slot s lives at (s / block_size, s % block_size).
 *     This is the layout the reference runner allocates
 *     (src/myvllm/engine/model_runner.py:311-314, views at :376-395).
 */
#ifndef MKV_H_
#define MKV_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MKV_ABI_VERSION 5

/* Element dtypes (torch.float32, torch.bfloat16, torch.float16,
 * torch.float8_e4m3fn, torch.int8).  FP8 is OCP e4m3fn: max 448, no
 * infinities, NaN = S.1111.111 (reference: model_runner.py:247,
 * attention.py:113).  INT8 holds the symmetric per-token-head codes of
 * kv_cache_dtype 'int8_per_token_head' (model_runner.py:242-244). */
#define MKV_DTYPE_F32 0
#define MKV_DTYPE_BF16 1
#define MKV_DTYPE_F16 2
#define MKV_DTYPE_FP8E4M3 3
#define MKV_DTYPE_I8 4

/* Granularity of the dequantisation scales of an FP8 / INT8 cache.
 *   PER_TENSOR:     k_scale / v_scale point at one fp32 each
 *                   (kv_cache_dtype 'fp8_per_tensor', model_runner.py:324-329).
 *   PER_TOKEN_HEAD: k_scale / v_scale are fp32 (num_blocks, block_size,
 *                   num_kv_heads) tensors in the pool's slot order: the scale
 *                   of slot s, kv head h is scale[s * num_kv_heads + h]
 *                   ('fp8_per_token_head' / 'int8_per_token_head',
 *                   model_runner.py:330-338). */
#define MKV_SCALE_PER_TENSOR 0
#define MKV_SCALE_PER_TOKEN_HEAD 1

/* Index dtypes for context_lens (the engine uses int64, model_runner.py:617;
 * the reference's micro-benchmarks use int32, benchmark_decoding.py:290). */
#define MKV_INDEX_I32 0
#define MKV_INDEX_I64 1

#define MKV_OK 0
#define MKV_ERR_NULL_POINTER (-1)
#define MKV_ERR_BAD_SHAPE (-2)
#define MKV_ERR_UNSUPPORTED_DTYPE (-3)
#define MKV_ERR_UNSUPPORTED_HEAD_DIM (-4)
#define MKV_ERR_UNSUPPORTED_GROUP (-5)
#define MKV_ERR_BAD_BLOCK_SIZE (-6)
#define MKV_ERR_WORKSPACE_TOO_SMALL (-7)
#define MKV_ERR_MISALIGNED (-8)
#define MKV_ERR_BAD_STRIDE (-9)
#define MKV_ERR_SCRATCH_LIMIT (-10)

/* ABI version of the loaded library (MKV_ABI_VERSION at build time). */
int mkv_abi_version(void);

/* Static, NUL-terminated description of a status code. */
const char* mkv_status_string(int status);

/*
 * K1: slot-mapped KV append.
 *
 * Replaces store_kvcache (attention.py:67-108, kernel :7-64) when
 * cache_dtype == in_dtype, and the per-tensor branch of store_kvcache_fp8
 * (attention.py:281-333, kernel :118-191) when cache_dtype ==
 * MKV_DTYPE_FP8E4M3.
 *
 * For every token t < num_tokens with slot = slot_mapping[t] >= 0 and
 * slot < num_blocks * block_size, row t of key (num_kv_heads * head_dim
 * elements starting at key + t * key_row_stride) is written to k_cache slot
 * `slot`, likewise value -> v_cache.  slot == -1 means "skip"; any other
 * negative or out-of-pool slot is skipped as well (never written).
 *
 * FP8 mode: q = clamp(float(x) / scale, -448, 448) rounded to e4m3fn with
 * round-to-nearest-even, scale = *k_scale (resp. *v_scale), a device fp32
 * scalar.  The divide is the IEEE-754 correctly rounded fp32 divide and NaN
 * inputs stay NaN, so the bytes equal torch's
 *   torch.clamp(x.float() / scale, -448, 448).to(torch.float8_e4m3fn).
 * With flags & MKV_APPEND_CALIBRATE_SENTINEL, a scale that holds the 1.0
 * "not yet calibrated" sentinel is first calibrated from all num_tokens rows
 * and written back, exactly as mkv_fp8_calibrate_per_tensor would, so one
 * call has store_kvcache_fp8's calibrate-once semantics
 * (attention.py:308-333).  That fallback re-reads the whole input in every
 * wavefront: run mkv_fp8_calibrate_per_tensor before the first append of a
 * tensor and use the flag for the later ones, where the sentinel normally
 * no longer occurs.  Without the flag the scales are only read.
 * Copy mode: the bytes are copied unchanged; k_scale/v_scale and flags are
 * ignored.
 *
 * Rows must be 16-byte aligned (base pointers and row strides).
 * in_dtype in {F32, BF16, F16}; cache_dtype == in_dtype or FP8E4M3.
 * head_dim * num_kv_heads must be a multiple of 16.
 */
#define MKV_APPEND_CALIBRATE_SENTINEL 1
int mkv_kv_append(const void* key, int64_t key_row_stride,
                  const void* value, int64_t value_row_stride,
                  void* k_cache, void* v_cache,
                  const int64_t* slot_mapping, int64_t num_tokens,
                  int num_kv_heads, int head_dim,
                  int block_size, int64_t num_blocks,
                  int in_dtype, int cache_dtype,
                  float* k_scale, float* v_scale, int flags,
                  void* stream);

/*
 * K1 with per-token-head quantisation.
 *
 * Replaces the per-token-head branch of store_kvcache_fp8
 * (attention.py:281-333, kernel :118-191, branch :166-181) when cache_dtype
 * == MKV_DTYPE_FP8E4M3 and store_kvcache_int8 (attention.py:246-276, kernel
 * :194-243) when cache_dtype == MKV_DTYPE_I8.
 *
 * Rows are selected as in mkv_kv_append (slot -1 or out of pool: skipped,
 * scales untouched).  For each written (token, kv head) with fp32 elements
 * x[0..head_dim) and amax = max |x| (NaN elements ignored, 0 if none left):
 *   FP8:  scale = amax > 0 ? amax / 448 : 1;  q = clamp(x / scale, +-448)
 *         rounded to e4m3fn (RNE; NaN stays NaN), as the per-tensor mode;
 *   INT8: scale = max(amax / 127, 1e-6);  y = x * (1 / scale);
 *         y += (y >= 0 ? 0.5 : -0.5);  q = trunc(minNum(maxNum(y, -128), 127))
 *         (round half away from zero; a NaN becomes -128).
 * Divisions are IEEE-754 correctly rounded fp32.  scale is written to
 * k_scale[slot * num_kv_heads + h] (v_scale likewise).
 *
 * head_dim a power of two in 16..1024; alignment as in mkv_kv_append.
 */
int mkv_kv_append_per_token_head(const void* key, int64_t key_row_stride,
                                 const void* value, int64_t value_row_stride,
                                 void* k_cache, void* v_cache,
                                 float* k_scale, float* v_scale,
                                 const int64_t* slot_mapping, int64_t num_tokens,
                                 int num_kv_heads, int head_dim,
                                 int block_size, int64_t num_blocks,
                                 int in_dtype, int cache_dtype, void* stream);

/*
 * Per-tensor FP8 calibration (attention.py:308-323), done on the device so
 * that no host synchronisation is needed.
 *
 * If *k_scale == 1.0f (the "not yet calibrated" sentinel that the runner
 * initialises with torch.ones, model_runner.py:327), it is replaced by
 *   round_in(max(round_in(amax|key|), round_in(1e-8)) / 448)
 * where round_in() rounds an fp32 value to in_dtype (RNE) and amax runs over
 * ALL num_tokens rows, including rows whose slot is -1.  Same for *v_scale.
 * A scale that is not exactly 1.0 is left untouched (calibrate once, then
 * freeze).  This is the reference's
 *   scale.fill_((x.abs().amax().clamp(min=1e-8) / 448.0).item())
 * evaluated in x's dtype.
 *
 * workspace: >= mkv_fp8_calibrate_workspace_size() bytes of device memory
 * that is zero before the first call; the kernel leaves it zero again.
 * Calls that share a workspace must be ordered on one stream.
 */
size_t mkv_fp8_calibrate_workspace_size(void);
int mkv_fp8_calibrate_per_tensor(const void* key, int64_t key_row_stride,
                                 const void* value, int64_t value_row_stride,
                                 int64_t num_tokens, int row_elems,
                                 int in_dtype,
                                 float* k_scale, float* v_scale,
                                 void* workspace, void* stream);

/*
 * K2: paged decode attention.
 *
 * Replaces paged_attention_decode (attention.py:895-950, kernel :517-646)
 * and paged_attention_decode_quantized (attention.py:1213-1268): the
 * per-tensor FP8 kernel (:953-1121) and the per-token-head FP8 / INT8 tile
 * kernel (:1124-1210).
 *
 * out[b, h, :] = softmax_t(sm_scale * q[b,h,:] . K_t) @ V_t over the tokens
 * t < context_lens[b] of sequence b whose logical block
 * block_tables[b, t / block_size] is a valid pool index (entries of -1 are
 * skipped), with K_t/V_t taken from kv head h / (num_heads / num_kv_heads).
 * Quantised caches are dequantised as code * scale: kv_scale_mode
 * MKV_SCALE_PER_TENSOR (FP8 only) uses *k_scale / *v_scale;
 * MKV_SCALE_PER_TOKEN_HEAD (FP8 or INT8) uses the scale of the token's slot
 * and kv head.  kv_scale_mode is ignored for F32/BF16/F16 caches.
 * A sequence with no visible token (context_lens[b] == 0) gets zeros.
 *
 * q, out: (batch, num_heads, head_dim), rows contiguous, row stride
 * q_batch_stride / out_batch_stride elements; out has q's dtype.
 * block_tables: int32 (batch, bt_stride) with max_blocks usable columns.
 * head_dim 128, num_heads / num_kv_heads in 1..16; or head_dim 64 (the
 * Llama-3.2-1B shape, main_llama32.py:29-34) with an even num_kv_heads and
 * num_heads / num_kv_heads in 1..8.  block_size a power of two >= 16.
 * q_dtype is F32, BF16 or F16 with any kv_dtype.
 *
 * split_tokens selects the schedule:
 *   0 = the library's choice from (batch, num_kv_heads, max_blocks,
 *       block_size, kv_dtype, kv_scale_mode): the workgroup route when the
 *       widest context the table allows gives each of its waves at most 128
 *       tokens, or at most 256 tokens when its waves also fill enough of
 *       the device (per-tensor FP8: 2 x CUs waves, BF16/F16: 6 x CUs;
 *       never for per-token-head scales; FP32: at most 512 tokens and
 *       2 x CUs waves); else stream-K (BF16/F16/FP8/INT8 KV, batch <= 8192),
 *       else split-K with a library-chosen split (mkv_paged_decode_route
 *       reports the choice);
 *   MKV_DECODE_STREAM = stream-K over 32-token tiles on a persistent grid,
 *       groups of num_kv_heads waves sharing each tile range, and a merge
 *       kernel (split-K where stream-K does not apply);
 *   MKV_DECODE_WORKGROUP = one workgroup per (sequence, KV head) whose waves
 *       split the sequence and merge in LDS (every KV format; no workspace,
 *       one launch);
 *   > 0 = split-K with that many tokens per work item (a multiple of 32).
 * Every route reads any block-table width (block-table entries are looked
 * up tile by tile).
 * workspace: >= mkv_paged_decode_workspace_size(...)
 * bytes with the same arguments (the size of the route those arguments
 * select: stream-K partial slots for the persistent grid, or split-K
 * partials, or 0; for an FP8 kv_dtype, which the query takes without a
 * scale mode, the larger of the per-tensor and the per-token-head route's);
 * calls that share a workspace must be ordered on one stream.
 */
#define MKV_DECODE_WORKGROUP (-1)
#define MKV_DECODE_STREAM (-2)
#define MKV_DECODE_ROUTE_STREAM 0
#define MKV_DECODE_ROUTE_SPLIT 1
#define MKV_DECODE_ROUTE_WORKGROUP 2
size_t mkv_paged_decode_workspace_size(int batch, int num_heads,
                                       int num_kv_heads, int max_blocks,
                                       int block_size, int head_dim,
                                       int kv_dtype, int split_tokens);

/* Tokens per split-K work item that mkv_paged_decode uses for these sizes
 * (split_tokens itself when it is > 0). */
int mkv_paged_decode_split_tokens(int batch, int num_kv_heads, int max_blocks,
                                  int block_size, int split_tokens);

/* The schedule mkv_paged_decode takes for these arguments on a device of
 * num_cus compute units (num_cus <= 0: the current device): one of
 * MKV_DECODE_ROUTE_STREAM / _SPLIT / _WORKGROUP, or a negative status for
 * an unsupported shape.  The reference has one decode entry and no schedule
 * (attention.py:895-950); this reports the library's choice for split_tokens
 * 0 (for an FP8 kv_dtype, with per-tensor scales: per-token-head scales may
 * take stream-K where this reports the workgroup route; INT8 is always per
 * token and head) and the route an explicit value selects. */
int mkv_paged_decode_route(int batch, int num_heads, int num_kv_heads,
                           int max_blocks, int block_size, int head_dim,
                           int kv_dtype, int split_tokens, int num_cus);
int mkv_paged_decode(void* out, int64_t out_batch_stride,
                     const void* q, int64_t q_batch_stride, int q_dtype,
                     const void* k_cache, const void* v_cache, int kv_dtype,
                     int64_t num_blocks,
                     const float* k_scale, const float* v_scale,
                     int kv_scale_mode,
                     const int32_t* block_tables, int64_t bt_stride,
                     int max_blocks,
                     const void* context_lens, int context_lens_dtype,
                     int batch, int num_heads, int num_kv_heads, int head_dim,
                     int block_size, float sm_scale, int split_tokens,
                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * K2 without a caller workspace, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  It has no counterpart in the reference.
 *
 * Same arguments and results as mkv_paged_decode (the same kernels and
 * schedule, so the outputs are bit-identical), minus workspace and
 * workspace_bytes: the partials live in a static per-device scratch array of
 * MKV_NOALLOC_SCRATCH_BYTES (32 MiB) that the library holds on each GPU it
 * runs on until the process ends.  The call allocates
 * and frees nothing.  When the route that mkv_paged_decode would take needs
 * more than that (see mkv_paged_decode_workspace_size; e.g. stream-K slots
 * for 16 query heads per KV head on 256 CUs), the library's choice
 * (split_tokens 0) takes the workgroup route instead, which needs no
 * workspace and agrees within rounding rather than bit for bit; an explicit
 * route returns MKV_ERR_SCRATCH_LIMIT before any launch.  Every call on one GPU shares that GPU's array: calls that overlap
 * on one GPU (different streams, or different host threads without
 * ordering) race and must be ordered by the caller.  The first call on a
 * device resolves the array's address on that device (make it outside graph
 * capture).
 */
#define MKV_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int mkv_paged_decode_noalloc(void* out, int64_t out_batch_stride,
                             const void* q, int64_t q_batch_stride, int q_dtype,
                             const void* k_cache, const void* v_cache, int kv_dtype,
                             int64_t num_blocks,
                             const float* k_scale, const float* v_scale,
                             int kv_scale_mode,
                             const int32_t* block_tables, int64_t bt_stride,
                             int max_blocks,
                             const void* context_lens, int context_lens_dtype,
                             int batch, int num_heads, int num_kv_heads, int head_dim,
                             int block_size, float sm_scale, int split_tokens,
                             void* stream);

/*
 * K3: causal prefill / extend attention over the paged cache.
 *
 * Replaces paged_attention_prefill_triton (attention.py:852-891, kernel
 * :704-847) and, with FP8 caches, fills the path that the reference leaves
 * unimplemented (attention.py:1702-1708).
 *
 * For query row i of sequence s (rows cu_seqlens_q[s] .. cu_seqlens_q[s+1])
 * and head h: visible = min(context_lens[s], positions[i] + 1); out[i, h] is
 * attention over logical tokens [0, visible) of sequence s, read through
 * block_tables as in K2 (-1 entries skipped).
 *
 * q, out: (total_q, num_heads, head_dim) contiguous.  positions: int64
 * (total_q).  cu_seqlens_q: int32 (num_seqs + 1).  kv_dtype F32 (the
 * reference engine's default, computed on the fp32 MFMA), BF16 or F16;
 * FP8E4M3 with kv_scale_mode MKV_SCALE_PER_TENSOR (k_scale / v_scale: one
 * fp32 each) or MKV_SCALE_PER_TOKEN_HEAD; INT8 with MKV_SCALE_PER_TOKEN_HEAD
 * (k_scale / v_scale: fp32 (num_blocks, block_size, num_kv_heads), as in
 * K2).  Per-token-head caches are an extension as well: the reference's
 * decode-path arithmetic (K scale on the score, V scale on P, the
 * denominator over the unscaled P) applied per key.  q_dtype F32, BF16 or
 * F16 with any kv_dtype; out has q's dtype.
 * workspace: >= mkv_paged_prefill_workspace_size(...) bytes (tile list).
 */
size_t mkv_paged_prefill_workspace_size(int num_seqs, int64_t total_q,
                                        int num_heads, int num_kv_heads);
int mkv_paged_prefill(void* out, const void* q, int q_dtype,
                      const void* k_cache, const void* v_cache, int kv_dtype,
                      int64_t num_blocks,
                      const float* k_scale, const float* v_scale,
                      int kv_scale_mode,
                      const int32_t* block_tables, int64_t bt_stride,
                      int max_blocks,
                      const void* context_lens, int context_lens_dtype,
                      const int32_t* cu_seqlens_q, const int64_t* positions,
                      int num_seqs, int64_t total_q,
                      int num_heads, int num_kv_heads, int head_dim,
                      int block_size, float sm_scale,
                      void* workspace, size_t workspace_bytes, void* stream);

/*
 * K3 on contiguous K/V: causal varlen attention over freshly projected
 * q/k/v (full prefill, every sequence starts at position 0).
 *
 * Replaces flash_attention_prefill (attention.py:446-514, kernel :336-443).
 * Row i of sequence s attends to rows cu_seqlens[s] .. i of k/v.
 * q, out: (total, num_heads, head_dim); k, v: (total, num_kv_heads,
 * head_dim); all contiguous and of one dtype (F32, BF16 or F16).
 */
size_t mkv_flash_prefill_workspace_size(int num_seqs, int64_t total,
                                        int num_heads, int num_kv_heads);
int mkv_flash_prefill(void* out, const void* q, const void* k, const void* v,
                      int dtype, const int32_t* cu_seqlens, int num_seqs,
                      int64_t total, int num_heads, int num_kv_heads,
                      int head_dim, float sm_scale,
                      void* workspace, size_t workspace_bytes, void* stream);

/*
 * K4: block-table gather, paged -> contiguous.
 *
 * The torch form of this gather is benchmark_decoding.py:166-178; every
 * paged kernel of the reference inlines it (attention.py:578-590, :787-798).
 * dst[b, t, :, :] = cache[block_tables[b, t / bs], t % bs, :, :] for
 * t < context_lens[b]; rows t >= context_lens[b] (up to max_len) and rows
 * whose block entry is -1 are zero-filled.  dst: (batch, max_len,
 * num_kv_heads, head_dim) in the cache dtype (any MKV_DTYPE_*: the bytes are
 * copied, quantised codes stay codes), contiguous.
 */
int mkv_gather_kv(void* dst, const void* cache, int dtype, int64_t num_blocks,
                  const int32_t* block_tables, int64_t bt_stride,
                  int max_blocks,
                  const void* context_lens, int context_lens_dtype,
                  int batch, int max_len, int num_kv_heads, int head_dim,
                  int block_size, void* stream);

/*
 * K6: fused producer — q/k RMSNorm + rotary embedding + KV append.
 *
 * Replaces, for one attention layer, the steps between the qkv projection
 * and the attention kernels: the q/k/v split and q_norm / k_norm of
 * Qwen3Attention.forward (qwen3.py:73-118; LayerNorm.rms_forward,
 * layernorm.py:16-24), the rotary embedding (rotary_embedding.py:100-109,
 * apply_rotary_pos_emb :4-26) and Attention.forward's contiguous copies and
 * append (attention.py:1654-1691: store_kvcache / store_kvcache_fp8 /
 * store_kvcache_int8).
 *
 * qkv: (num_tokens, qkv_row_stride) rows holding q (num_heads * head_dim),
 * then k and v (num_kv_heads * head_dim each), in in_dtype.  For each token t
 * and q / k head, with x the head's elements in fp32:
 *   norm (if the weight pointer is non-null):
 *     y = round_in(x / sqrt(sum(x^2) / head_dim + eps) * weight)
 *   rotary at p = positions[t], c = cos_sin_cache[p, i], s =
 *     cos_sin_cache[p, head_dim/2 + i] for i < head_dim/2 (NeoX halves):
 *     out[i] = y[i]*c - y[i + D/2]*s,  out[i + D/2] = y[i]*s + y[i + D/2]*c
 *   rounded to out_dtype (fp32 products and sums, no fused multiply-add).
 * q_out (num_tokens, num_heads, head_dim) and, if non-null, k_out
 * (num_tokens, num_kv_heads, head_dim) receive the rotated q / k in
 * out_dtype.  The rotated k and the raw v of every token with slot =
 * slot_mapping[t] in [0, num_blocks * block_size) are appended as
 * mkv_kv_append (cache_dtype = a float type: cast on store; FP8E4M3 with
 * kv_scale_mode PER_TENSOR, honouring flags as mkv_kv_append, where the
 * 1.0-sentinel calibration uses this call's rotated k / raw v) or
 * mkv_kv_append_per_token_head (FP8E4M3 or I8 with PER_TOKEN_HEAD) would
 * append them.  slot_mapping NULL: nothing is appended (the caches and
 * scales may be NULL then).  A position outside [0, max_position) gives NaN
 * outputs.
 *
 * head_dim a power of two in 32..1024; in / out / cos_sin / weight dtypes
 * F32, BF16 or F16; 16-byte aligned pointers and qkv row stride.
 */
int mkv_qkv_norm_rope_append(const void* qkv, int64_t qkv_row_stride,
                             int in_dtype, int64_t num_tokens,
                             int num_heads, int num_kv_heads, int head_dim,
                             const void* q_norm_weight,
                             const void* k_norm_weight,
                             int norm_weight_dtype, float eps,
                             const void* cos_sin_cache, int cos_sin_dtype,
                             int64_t max_position, const int64_t* positions,
                             void* q_out, void* k_out, int out_dtype,
                             void* k_cache, void* v_cache, int cache_dtype,
                             int kv_scale_mode, float* k_scale, float* v_scale,
                             const int64_t* slot_mapping, int block_size,
                             int64_t num_blocks, int flags, void* stream);

/*
 * K6 + K2 in one launch for a decode step: one layer's producer step for the
 * one new token of each sequence, then the decode attention over the cache
 * that holds it.
 *
 * Replaces, for a decode step, mkv_qkv_norm_rope_append over the batch's
 * qkv rows (token b of sequence b; Qwen3Attention.forward, qwen3.py:73-118,
 * and the append of Attention.forward, attention.py:1654-1691) followed by
 * mkv_paged_decode on its q (paged_attention_decode_quantized,
 * attention.py:1213-1268), and gives the same bits as that pair: the same
 * cache bytes and scales, and out equal to the decode of the producer's q
 * with out_dtype as its dtype.  The arguments are those of the two calls
 * (num_tokens = batch, q_out / k_out absent, split_tokens
 * MKV_DECODE_WORKGROUP: this runs the workgroup route).  slot_mapping[b]
 * (required; -1 or out of the pool: nothing is appended for row b) must be
 * the cache row of position context_lens[b] - 1 of sequence b, as the
 * reference's prepare_decode builds it (model_runner.py:621-640), and no
 * other row of the batch may read it: the attention sees the appended row
 * at that position only.
 * Supported: kv_dtype FP8E4M3 with kv_scale_mode PER_TENSOR; F16; BF16,
 * or FP8E4M3 / I8 with kv_scale_mode PER_TOKEN_HEAD (k_scale / v_scale the
 * per-slot scales, written for the appended rows), with out_dtype BF16;
 * head_dim 128; num_heads / num_kv_heads <= 8 (MKV_ERR_UNSUPPORTED_DTYPE /
 * MKV_ERR_UNSUPPORTED_HEAD_DIM / MKV_ERR_UNSUPPORTED_GROUP otherwise,
 * before any launch: run the two calls).  flags as mkv_qkv_norm_rope_append
 * (the 1.0-sentinel calibration uses this call's rows; it applies to
 * per-tensor FP8 only; 16-bit caches take no scales).
 */
int mkv_qkv_norm_rope_append_decode(
    void* out, int64_t out_batch_stride, int out_dtype,
    const void* qkv, int64_t qkv_row_stride, int in_dtype,
    const void* q_norm_weight, const void* k_norm_weight,
    int norm_weight_dtype, float eps,
    const void* cos_sin_cache, int cos_sin_dtype, int64_t max_position,
    const int64_t* positions,
    void* k_cache, void* v_cache, int kv_dtype, int64_t num_blocks,
    float* k_scale, float* v_scale, int kv_scale_mode,
    const int64_t* slot_mapping, int flags,
    const int32_t* block_tables, int64_t bt_stride, int max_blocks,
    const void* context_lens, int context_lens_dtype,
    int batch, int num_heads, int num_kv_heads, int head_dim,
    int block_size, float sm_scale, void* stream);

/*
 * Decode-step metadata on the device.
 *
 * Replaces the per-step host loop of ModelRunner.prepare_decode
 * (model_runner.py:621-640) and the graph-buffer copies of run_model
 * (:695-701).  The caller keeps, per batch row b < rows, the sequence length
 * seq_lens[b] (int64; <= 0 = inactive row) and its block table row
 * block_tables[b, 0 .. max_blocks) resident on the device.  For each row:
 *   active (seq_lens[b] > 0):  L = seq_lens[b] + increment;
 *       seq_lens[b] = context_lens[b] = L;
 *       slot_mapping[b] = block_tables[b, (L-1) / block_size] * block_size
 *                         + (L-1) % block_size
 *       (-1 if that entry is -1, outside the pool or past max_blocks);
 *   inactive:  seq_lens[b] = context_lens[b] = 0, slot_mapping[b] = -1
 *       (the append skips the row and the decode writes zeros: the padded
 *       rows of a captured batch).
 * With increment == 1 the call advances every active sequence by the token
 * decoded this step (len(seq) in the reference); with 0 it only derives the
 * metadata.  context_lens may alias seq_lens.  block_size a power of two.
 */
int mkv_decode_metadata(int64_t* seq_lens, int64_t* context_lens,
                        int64_t* slot_mapping, const int32_t* block_tables,
                        int64_t bt_stride, int max_blocks, int64_t num_blocks,
                        int block_size, int rows, int increment, void* stream);

/*
 * Decoder-layer row operations of the end-to-end engine (mkv.engine), one
 * HBM pass each.
 *
 * mkv_rmsnorm replaces LayerNorm.rms_forward / residual_rms_forward
 * (layernorm.py:16-33).  x, out: (rows, hidden) contiguous; weight:
 * (hidden,).  If residual is non-NULL it is updated in place to
 * round(x + residual) and normalised; otherwise x is.  With h the row being
 * normalised: out = round(h * weight / sqrt(sum(h^2) / hidden + eps)), fp32
 * arithmetic, one rounding to dtype.  hidden a multiple of 8, <= 2048;
 * 16-byte aligned pointers.
 *
 * mkv_silu_mul replaces SiluAndMul (activation.py:16-19): x rows of
 * 2 * inter elements (row stride x_row_stride >= 2 * inter), out (rows,
 * inter) contiguous, out = round(silu(x[:, :inter]) * x[:, inter:]) with
 * silu(a) = a / (1 + exp(-a)) in fp32.  inter a multiple of 8.
 *
 * dtype F32, BF16 or F16.
 */
int mkv_rmsnorm(void* out, void* residual, const void* x, const void* weight,
                int64_t rows, int hidden, float eps, int dtype, void* stream);
int mkv_silu_mul(void* out, const void* x, int64_t x_row_stride, int64_t rows,
                 int inter, int dtype, void* stream);

/* ------------------------------------------------------------------------
 * Measurement helper (no counterpart in the reference; for benchmarks).
 *
 * mkv_stream_read_probe reads `bytes` (a multiple of 16) from the 16-byte
 * aligned device buffer `buf` once, with the non-temporal 16-byte loads the
 * decode kernels use for KV, in `grid` (<= 2^20) workgroups of 256 threads
 * (grid-stride, up to 16 loads in flight per lane), and writes one XOR checksum
 * dword per wavefront to `sink` (mkv_stream_read_probe_sink_words(grid)
 * words).  Its time gives the read rate a plain streaming kernel reaches on
 * the GPU, the measured ceiling next to the datasheet peak.
 */
size_t mkv_stream_read_probe_sink_words(int grid);
int mkv_stream_read_probe(const void* buf, int64_t bytes, uint32_t* sink, int grid,
                          void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MKV_H_ */
