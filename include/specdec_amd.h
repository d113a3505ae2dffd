/*
 * specdec_amd.h — C ABI of the MI355X (gfx950) decode hot path.
 *
 * The library `libspecdec_amd.so` exports exactly the functions below. Every
 * entry point takes plain device pointers, element strides and sizes, and a
 * `hipStream_t` passed as `void*` (NULL = the legacy default stream). Nothing
 * here allocates, frees or synchronises: output buffers and workspaces are
 * owned by the caller, and every launch is enqueued on the given stream, so
 * calls can be captured into a HIP graph and issued from several streams at
 * once (each call uses only the workspace it is handed).
 *
 * Return value: SD_OK (0) or a nonzero `sd_status`; the message of the last
 * failure on the calling thread is returned by `sd_last_error()`.
 *
 * Dtype codes: SD_BF16, SD_F16 for activations/caches; scales may also be
 * SD_F32. Strides are in ELEMENTS of the tensor they describe.
 *
 * Bounds: every stride must lie within +-2^40 elements (W8A16 strides are
 * non-negative), and sizes past what one GPU could hold are refused before any
 * arithmetic on them (sequence and row counts below 2^31, page pools below
 * 2^32 blocks, context bounds below 2^30 keys). A refused call returns
 * SD_ERR_VALUE or SD_ERR_UNSUPPORTED and launches nothing; a workspace query
 * for such sizes returns SIZE_MAX.
 */
#ifndef SPECDEC_AMD_H
#define SPECDEC_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SD_ABI_VERSION 2

typedef enum sd_status {
  SD_OK = 0,
  SD_ERR_VALUE = 1,       /* bad argument: the reference raises AssertionError/ValueError */
  SD_ERR_UNSUPPORTED = 2, /* valid but not implemented shape/dtype: reference TORCH_CHECK */
  SD_ERR_WORKSPACE = 3,   /* workspace NULL or smaller than the *_workspace_size() query */
  SD_ERR_HIP = 4          /* a HIP launch reported an error */
} sd_status;

typedef enum sd_dtype { SD_BF16 = 0, SD_F16 = 1, SD_F32 = 2 } sd_dtype;

/* ABI version compiled into the library (== SD_ABI_VERSION of its header). */
int sd_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* sd_last_error(void);

/*
 * KV-cache slot write.
 * Replaces `store_kvcache` + `store_kvcache_kernel`
 * (nanovllm/layers/attention.py:10-40): for every token i with
 * s = slot_mapping[i] != -1, row i of key/value (num_kv_heads x head_dim) is
 * copied bit-for-bit to cache position (s / block_size, s % block_size).
 * Slots outside [0, num_blocks*block_size) are skipped like -1 (the reference
 * leaves them undefined). Works for any 2- or 4-byte element type.
 *   key/value  : (num_tokens, num_kv_heads, head_dim), head_dim contiguous
 *   k/v_cache  : (num_blocks, block_size, num_kv_heads, head_dim) by strides
 */
int sd_store_kvcache(const void* key, int64_t key_stride_tok, int64_t key_stride_head,
                     const void* value, int64_t value_stride_tok, int64_t value_stride_head,
                     void* k_cache, void* v_cache, int64_t cache_stride_block,
                     int64_t cache_stride_pos, int64_t cache_stride_head,
                     const int32_t* slot_mapping, int64_t num_tokens, int32_t num_kv_heads,
                     int32_t head_dim, int32_t block_size, int64_t num_blocks,
                     int32_t elem_bytes, void* stream);

/*
 * Bytes of fp32 split-KV workspace that sd_paged_attention needs for these
 * sizes on the CURRENT device (the work is divided among a number of
 * workgroups that follows the device's compute-unit count).
 *   max_ctx     : block_table width * block_size (static bound, no host sync)
 *   num_splits  : 0 = library default (one resident set of workgroups shares
 *                 all keys), n > 0 = about n workgroups per (sequence, kv head)
 */
size_t sd_paged_attention_workspace_size(int32_t num_seqs, int32_t max_qlen,
                                         int32_t num_q_heads, int32_t num_kv_heads,
                                         int32_t head_dim, int64_t max_ctx,
                                         int32_t num_splits);

/*
 * Paged decode / speculative-verify attention (GQA, split-KV).
 * Replaces the decode call `flash_attn_with_kvcache(q, k_cache, v_cache,
 * cache_seqlens, block_table, softmax_scale, causal=True)`
 * (nanovllm/layers/attention.py:71-81), the paged verify call
 * `flash_attn_varlen_func(..., causal=True, block_table)` (attention.py:64-70
 * with model_runner.py:492-584), and the standalone kernels
 * `paged_decode_attention` (nanovllm/kernels/paged_decode_attn.py:352-469) and
 * `paged_decode_cuda` (nanovllm/kernels/paged_decode_attn_cuda.cu:1388-1453).
 *
 * Sequence b has L_b keys (context_lens[b], or cu_seqlens_k[b+1]-cu_seqlens_k[b]
 * when context_lens is NULL) and n_b query rows starting at token
 * cu_seqlens_q[b] (or n_b = 1 at token b when cu_seqlens_q is NULL). Query row
 * i of sequence b attends keys [0, L_b - n_b + i] (bottom-right causal; for
 * n_b = 1 that is all L_b keys). Key position p is read from page
 * block_table[b, p / block_size], row p % block_size. A row with no visible
 * key (L_b = 0 padding rows) produces zeros. Query rows at or beyond total_q
 * (the first dimension of q and out) are never read or written, and L_b is
 * clamped into [0, max_blocks_per_seq * block_size].
 *   q      : (total_q, num_q_heads, head_dim)
 *   out    : (total_q, num_q_heads, head_dim), same dtype as q
 *   caches : (num_blocks, block_size, num_kv_heads, head_dim) by strides
 *            (interleaved or head-major page layouts both work)
 * Supported: head_dim 128, dtype bf16/f16, (num_q_heads/num_kv_heads) *
 * max_qlen <= 32. Page ids are clamped into [0, num_blocks).
 * workspace: >= sd_paged_attention_workspace_size(...) bytes, 16-byte
 * aligned, queried on the same device. num_splits: as in that query.
 * Keys are divided evenly among the workgroups across all (sequence, kv head)
 * pairs (no host sync: the kernels read context_lens themselves); a second
 * kernel merges the partial softmax states of pairs that several workgroups
 * shared and writes zeros for sequences without keys.
 */
int sd_paged_attention(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                       const void* k_cache, const void* v_cache, int64_t cache_stride_block,
                       int64_t cache_stride_pos, int64_t cache_stride_head, int64_t num_blocks,
                       int32_t block_size, const int32_t* block_table, int64_t bt_stride,
                       int32_t max_blocks_per_seq, const int32_t* context_lens,
                       const int32_t* cu_seqlens_k, const int32_t* cu_seqlens_q,
                       int32_t max_qlen, int64_t total_q, int32_t num_seqs, int32_t num_q_heads,
                       int32_t num_kv_heads, int32_t head_dim, float scale, int32_t dtype,
                       void* out, int64_t out_stride_tok, int64_t out_stride_head,
                       void* workspace, size_t workspace_bytes, int32_t num_splits,
                       void* stream);

/*
 * sd_paged_attention without the workspace arguments, allocating nothing: the
 * split-KV workspace is the library's static device scratch (one per device,
 * SD_NOALLOC_SCRATCH_BYTES). The scratch is part of the library's code
 * object: it is reserved on every device where the library's kernels load,
 * for any user of the library, whether or not this entry is ever called, and
 * held until the process ends. Its device address is looked up once per
 * device (hipGetSymbolAddress, on the first call with that device current)
 * and kept: after hipDeviceReset, or anything else that reloads the library's
 * code object on a device, that address is stale, and this entry must not be
 * called again in the process. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same kernels, plan and results as
 * sd_paged_attention with a workspace (bit for bit). Sizes whose workspace
 * (sd_paged_attention_workspace_size) exceeds the scratch return
 * SD_ERR_UNSUPPORTED. Every call on a device shares that device's scratch:
 * calls that overlap in time on one device (two streams, two threads) race and
 * must be ordered by the caller. Nothing needs clearing between calls (every
 * partial the merge reads is written earlier in the same call).
 */
#define SD_NOALLOC_SCRATCH_BYTES (32u << 20)
int sd_paged_attention_noalloc(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                               const void* k_cache, const void* v_cache,
                               int64_t cache_stride_block, int64_t cache_stride_pos,
                               int64_t cache_stride_head, int64_t num_blocks,
                               int32_t block_size, const int32_t* block_table,
                               int64_t bt_stride, int32_t max_blocks_per_seq,
                               const int32_t* context_lens, const int32_t* cu_seqlens_k,
                               const int32_t* cu_seqlens_q, int32_t max_qlen,
                               int64_t total_q, int32_t num_seqs, int32_t num_q_heads,
                               int32_t num_kv_heads, int32_t head_dim, float scale,
                               int32_t dtype, void* out, int64_t out_stride_tok,
                               int64_t out_stride_head, int32_t num_splits, void* stream);

/*
 * Same arguments as sd_paged_attention, but only the split-KV main kernel
 * runs: `out` receives the rows of (sequence, kv head) pairs that one
 * workgroup covered and the workspace the partial (m, l, acc) of the others;
 * rows of sequences without keys are left untouched. Measurement twin of
 * `paged_decode_cuda_partial` (nanovllm/kernels/paged_decode_attn_cuda.cu:1558-1593).
 */
int sd_paged_attention_partial(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                               const void* k_cache, const void* v_cache,
                               int64_t cache_stride_block, int64_t cache_stride_pos,
                               int64_t cache_stride_head, int64_t num_blocks,
                               int32_t block_size, const int32_t* block_table,
                               int64_t bt_stride, int32_t max_blocks_per_seq,
                               const int32_t* context_lens, const int32_t* cu_seqlens_k,
                               const int32_t* cu_seqlens_q, int32_t max_qlen,
                               int64_t total_q, int32_t num_seqs, int32_t num_q_heads,
                               int32_t num_kv_heads,
                               int32_t head_dim, float scale, int32_t dtype, void* out,
                               int64_t out_stride_tok, int64_t out_stride_head,
                               void* workspace, size_t workspace_bytes,
                               int32_t num_splits, void* stream);

/*
 * Same arguments as sd_paged_attention, but only the merge kernel runs, over
 * the workspace that a sd_paged_attention_partial call with the same
 * arguments filled (stream-ordered before it): the rows of shared pairs and
 * the zero rows of sequences without keys are written to `out`. Together the
 * two calls give sd_paged_attention's result. Measurement twin of
 * `paged_decode_cuda_combine` (nanovllm/kernels/paged_decode_attn_cuda.cu:1544-1555).
 */
int sd_paged_attention_combine(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                               const void* k_cache, const void* v_cache,
                               int64_t cache_stride_block, int64_t cache_stride_pos,
                               int64_t cache_stride_head, int64_t num_blocks,
                               int32_t block_size, const int32_t* block_table,
                               int64_t bt_stride, int32_t max_blocks_per_seq,
                               const int32_t* context_lens, const int32_t* cu_seqlens_k,
                               const int32_t* cu_seqlens_q, int32_t max_qlen,
                               int64_t total_q, int32_t num_seqs, int32_t num_q_heads,
                               int32_t num_kv_heads, int32_t head_dim, float scale,
                               int32_t dtype, void* out, int64_t out_stride_tok,
                               int64_t out_stride_head, void* workspace,
                               size_t workspace_bytes, int32_t num_splits, void* stream);

/*
 * Read-only floor of the main kernel: same arguments and grid as
 * sd_paged_attention_partial, issuing exactly its K/V and q loads (same runs,
 * order and prefetch) with no math; nothing is written to `out`, and the
 * workspace is used only as a never-taken sink that keeps the loads. Its time
 * is the access pattern's own, the floor the main kernel can approach.
 * Measurement twin of `paged_decode_readonly_kernel` / `read_only`
 * (nanovllm/kernels/paged_decode_attn_cuda.cu:654-705,1244-1281).
 */
int sd_paged_attention_floor(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                             const void* k_cache, const void* v_cache,
                             int64_t cache_stride_block, int64_t cache_stride_pos,
                             int64_t cache_stride_head, int64_t num_blocks, int32_t block_size,
                             const int32_t* block_table, int64_t bt_stride,
                             int32_t max_blocks_per_seq, const int32_t* context_lens,
                             const int32_t* cu_seqlens_k, const int32_t* cu_seqlens_q,
                             int32_t max_qlen, int64_t total_q, int32_t num_seqs,
                             int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                             float scale, int32_t dtype, void* out, int64_t out_stride_tok,
                             int64_t out_stride_head, void* workspace, size_t workspace_bytes,
                             int32_t num_splits, void* stream);

/*
 * The box's streaming-read ceiling: one grid-stride pass of 16-byte
 * nontemporal loads over `bytes` (a positive multiple of 16) at `src`
 * (16-byte aligned), with `workgroups` workgroups of 256 threads (<= 0: six
 * per CU). Nothing is written except, practically never, one word of `sink`
 * (4-byte aligned device memory), which keeps the loads alive. The bench
 * divides the bytes by its time to get the bandwidth this GPU actually
 * reaches, the second denominator beside the 8 TB/s data-sheet peak. No
 * counterpart entry in the reference, which measured its own ceiling with a
 * plain device copy (nanovllm/kernels/README.md:27-35); the kernels here read
 * far more than they write, so the ceiling that bounds them is a read.
 */
int sd_stream_read(const void* src, int64_t bytes, void* sink, int32_t workgroups,
                   void* stream);

/*
 * store_kvcache + paged attention in one launch: the decode / verify layer call
 * `Attention.forward` (nanovllm/layers/attention.py:59-82: store_kvcache of the
 * new rows, then flash_attn_with_kvcache or the paged flash_attn_varlen_func).
 * Arguments as sd_paged_attention, plus the new rows: key/value
 * (total_q, num_kv_heads, head_dim) and slot_mapping (total_q,), row t being
 * query row t's key/value (decode: one per sequence; verify: the n_b rows of
 * sequence b). Result: bit for bit the same cache as sd_store_kvcache, and the
 * output of sd_paged_attention afterwards up to rounding (within the attention
 * tolerance), PROVIDED that the new rows of sequence b are its last n_b keys in
 * block_table order with slot -1 or the slot of that position — what
 * prepare_decode / prepare_verify and the draft proposer produce
 * (model_runner.py:466-482,522-548, draft_proposer.py:527-550). The main
 * kernel attends over the cached keys; the second (combine) launch adds the
 * new keys from key/value (fp32 scores) and copies the rows into the cache, so
 * no kernel waits for the store. num_seqs == 0 with total_q > 0 only stores.
 */
int sd_paged_attention_store(const void* key, int64_t key_stride_tok, int64_t key_stride_head,
                             const void* value, int64_t value_stride_tok,
                             int64_t value_stride_head, const int32_t* slot_mapping,
                             const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                             void* k_cache, void* v_cache, int64_t cache_stride_block,
                             int64_t cache_stride_pos, int64_t cache_stride_head,
                             int64_t num_blocks, int32_t block_size, const int32_t* block_table,
                             int64_t bt_stride, int32_t max_blocks_per_seq,
                             const int32_t* context_lens, const int32_t* cu_seqlens_k,
                             const int32_t* cu_seqlens_q, int32_t max_qlen, int64_t total_q,
                             int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                             int32_t head_dim, float scale, int32_t dtype, void* out,
                             int64_t out_stride_tok, int64_t out_stride_head, void* workspace,
                             size_t workspace_bytes, int32_t num_splits, void* stream);

/*
 * Bytes of workspace that sd_w8a16_linear needs for this shape. Always 0 in
 * this implementation (one launch; K splits are reduced inside a workgroup);
 * the query and the workspace arguments stay in the ABI so callers need not
 * change if a shape ever needs scratch memory.
 */
size_t sd_w8a16_workspace_size(int64_t M, int64_t N, int64_t K, int32_t group_size);

/*
 * W8A16 weight-only linear: y = x @ (w * scale)^T (+ bias).
 * Replaces `int8_linear` with `_int8_dequant_gemm_kernel` and
 * `_splitk_reduce_kernel` (nanovllm/layers/quant.py:165-310).
 *   x     : (M, K) dtype (bf16/f16), row stride x_stride_m, K contiguous
 *   w     : (N, K) int8, row stride w_stride_n, K contiguous
 *   scale : (N,) when group_size == 0 (per channel), else (N, K/group_size)
 *           row-major; scale_dtype bf16/f16/f32
 *   bias  : (N,) dtype or NULL
 *   y     : (M, N) dtype, row stride y_stride_m
 * Dequantization is fused (int8 -> fp in registers, fp32 accumulation, scale
 * applied to the fp32 accumulator). One or two activation rows with a
 * per-channel scale on weights up to 32 MiB (M * ceil(K / 1024) <= 4) stream
 * whole weight rows through fp32 FMAs, and so does one row on larger weights
 * (the lm_head), with batches of 4 rows dealt to the waves in turn; other
 * shapes run the MFMA kernel (the SiLU and RMSNorm forms below follow the
 * same rule). Supported: K % 64 == 0,
 * group_size 0 or a multiple of 64 dividing K; N < 2^24 rows, a row stride
 * below 2^24 bytes and N * w_stride_n < 2^32 bytes (the MFMA kernel forms a
 * row's byte offset with one 24 x 24-bit multiply-add; SD_ERR_UNSUPPORTED
 * otherwise). `workspace` may be NULL.
 * y may share no byte with x (SD_ERR_VALUE): other workgroups still read x
 * while one writes y.
 */
int sd_w8a16_linear(const void* x, int64_t x_stride_m, const int8_t* w, int64_t w_stride_n,
                    const void* scale, int32_t scale_dtype, int32_t group_size,
                    const void* bias, void* y, int64_t y_stride_m, int64_t M, int64_t N,
                    int64_t K, int32_t dtype, void* workspace, size_t workspace_bytes,
                    void* stream);

/*
 * Measurement twin of sd_w8a16_linear (per-channel scale): the same plan,
 * grid, activation staging, weight loads and prefetch, with every loaded
 * word folded into a register in place of the dequantization, the math and
 * the epilogue. y is not written (a store guarded by a condition on the
 * loaded data that is practically never true keeps the loads alive). Its time
 * is what the kernel's access pattern alone costs. The W8A16 counterpart of
 * sd_paged_attention_floor; the reference has no such twin for its int8
 * kernel (its attention twin is paged_decode_readonly_kernel,
 * nanovllm/kernels/paged_decode_attn_cuda.cu:654-705).
 */
int sd_w8a16_floor(const void* x, int64_t x_stride_m, const int8_t* w, int64_t w_stride_n,
                   const void* scale, int32_t scale_dtype, const void* bias, void* y,
                   int64_t y_stride_m, int64_t M, int64_t N, int64_t K, int32_t dtype,
                   void* stream);

/*
 * SiluAndMul fused into the W8A16 linear: y = (bf16(bf16(silu(g)) * u)) @
 * (w * scale)^T (+ bias) with g = gate_up[m, 0:K] and u = gate_up[m, K:2K],
 * the MLP's act_fn followed by down_proj (nanovllm/layers/activation.py:6-11,
 * models/qwen3.py Qwen3MLP.forward). No counterpart entry in the reference:
 * the fusion saves the SiluAndMul launch and its round trip through memory.
 * The activation equals sd_silu_mul's output bit for bit, so y equals
 * sd_silu_mul followed by sd_w8a16_linear. gate_up: (M, >= 2K) dtype, row
 * stride gate_up_stride_m, sharing no byte with y; the rest as
 * sd_w8a16_linear (no workspace). On the
 * row-streaming path (one or two rows, see sd_w8a16_linear) each wave forms
 * the SiLU of its columns once; otherwise it is computed once per workgroup
 * while its activation rows are staged in LDS, which holds while
 * min(M, 16) * (2 K + 16) <= 33,024 bytes; beyond that the result is the same
 * but each wave recomputes the SiLU of its operands, slower than the two
 * separate calls.
 */
int sd_w8a16_silu_linear(const void* gate_up, int64_t gate_up_stride_m, const int8_t* w,
                         int64_t w_stride_n, const void* scale, int32_t scale_dtype,
                         int32_t group_size, const void* bias, void* y, int64_t y_stride_m,
                         int64_t M, int64_t N, int64_t K, int32_t dtype, void* stream);

/*
 * add + RMSNorm fused into the W8A16 linear: y = norm(x [+ residual]) @
 * (w * scale)^T (+ bias), with norm the sd_rmsnorm row above (the decoder
 * layer's input_layernorm / post_attention_layernorm followed by qkv_proj /
 * gate_up_proj, models/qwen3.py Qwen3DecoderLayer.forward). No counterpart
 * entry in the reference: the fusion saves the RMSNorm launch and its round
 * trip through memory. The normalised row equals sd_rmsnorm's out bit for bit,
 * so y equals sd_rmsnorm followed by sd_w8a16_linear; with a residual,
 * residual_out (may be NULL) receives bf16(x + residual) as sd_rmsnorm's
 * residual_out does, written by one workgroup per row block. residual_out and
 * y may share no byte with x, residual or each other (other workgroups still
 * read the inputs): SD_ERR_VALUE. On the
 * row-streaming path (one or two rows, see sd_w8a16_linear) every wave forms
 * the norm of its columns; otherwise each workgroup normalises its activation
 * rows, one after another, while staging them in LDS. The form pays for a few
 * rows (decode), not for many (break-even near M = 5 on MI355X). A block that
 * does not fit the staging LDS (min(M, 16) (2 K + 16) > 33,024 bytes is never
 * promised) returns SD_ERR_UNSUPPORTED and the caller runs the two calls.
 *   x, residual, residual_out: (M, K) dtype, 16-byte aligned rows;
 *   norm_weight: (K,) dtype; K % 8 == 0, K <= 8192; the rest as
 *   sd_w8a16_linear (no workspace).
 */
int sd_w8a16_rmsnorm_linear(const void* x, int64_t x_stride_m, const void* residual,
                            int64_t residual_stride_m, void* residual_out,
                            int64_t residual_out_stride_m, const void* norm_weight, float eps,
                            const int8_t* w, int64_t w_stride_n, const void* scale,
                            int32_t scale_dtype, int32_t group_size, const void* bias, void* y,
                            int64_t y_stride_m, int64_t M, int64_t N, int64_t K, int32_t dtype,
                            void* stream);

/*
 * The MLP's gate_up projection with SiluAndMul applied to its output: for
 * weight w (N, K) = [gate rows; up rows] (N = 2 I),
 *   y[m, i] = bf16(bf16(silu(g)) * u), g = (a @ w[i]^T) * scale[i],
 *   u = (a @ w[I + i]^T) * scale[I + i], each rounded to dtype first,
 * with a = x, or a = RMSNorm(x [+ residual]) when norm_weight is not NULL
 * (the sd_rmsnorm row; residual_out receives bf16(x + residual) as there).
 * The layer's post_attention_layernorm, gate_up_proj and act_fn
 * (models/qwen3.py Qwen3MLP.forward, layers/activation.py:6-11) in one launch;
 * no counterpart entry in the reference. y equals sd_w8a16_rmsnorm_linear (or
 * sd_w8a16_linear) followed by sd_silu_mul bit for bit. On the row-streaming
 * path (one or two rows, M * ceil(K / 1024) <= 4, per-channel scale, at most
 * 32 MiB of weights, N even) a wave streams gate row i together with up row
 * I + i; on the K-split path of sd_w8a16_linear (narrow layers, per-channel
 * scale, N a multiple of 32) a workgroup takes gate tile g and up tile g with
 * the plain projection's K split, so the sums are the projection's own. The
 * down projection then reads the activated rows with no SiLU of its own.
 * Other shapes return SD_ERR_UNSUPPORTED (the caller runs the two calls).
 * y: (M, N / 2) dtype, sharing no byte with x, residual or residual_out.
 */
int sd_w8a16_gate_up_silu(const void* x, int64_t x_stride_m, const void* residual,
                          int64_t residual_stride_m, void* residual_out,
                          int64_t residual_out_stride_m, const void* norm_weight, float eps,
                          const int8_t* w, int64_t w_stride_n, const void* scale,
                          int32_t scale_dtype, const void* bias, void* y, int64_t y_stride_m,
                          int64_t M, int64_t N, int64_t K, int32_t dtype, void* stream);

/*
 * Symmetric int8 weight quantization, the producer of the W8A16 format:
 * `quantize_weight` (nanovllm/layers/quant.py:123-148) and the offline
 * converter's `quantize_tensor` (scripts/quantize_int8.py:53-83). Per row and
 * group (group_size columns, or the whole row when group_size == 0), in fp32:
 * scale = max(max|w| / 127, 1e-8); q = clamp(round_half_even(w / scale), -127,
 * 127). Writes q (N, K) int8 (row stride q_stride) and scale (N, K / group)
 * bf16 row-major (the fp32 scale rounded to nearest even, after q).
 *   w: (N, K) bf16/f16/f32, 16-byte aligned rows; K and the group size
 *   multiples of 8, the group size dividing K.
 */
int sd_quantize_int8(const void* w, int64_t w_stride, int32_t dtype, int8_t* q, int64_t q_stride,
                     void* scale, int64_t N, int32_t K, int32_t group_size, void* stream);

/* ---------------------------------------------------------------------------
 * Neighbours of the draft step (the row-wise work of a Qwen3 decoder step
 * between the attention and linear launches). Eager-torch rounding: fp32
 * arithmetic, a 16-bit rounding wherever the module converts to the
 * activation dtype, no fused multiply-add where the module has none.
 * ------------------------------------------------------------------------- */

/*
 * RMSNorm.forward (nanovllm/layers/layernorm.py:16-47). Per row of `hidden`:
 *   residual == NULL: out = bf16(bf16(x * r) * weight), r = rsqrt(mean(x^2) + eps)
 *   residual != NULL: s = x + residual (fp32); residual_out = bf16(s);
 *                     out = bf16(bf16(s * r) * weight), r from s
 * x/residual/out/residual_out: (rows, hidden) dtype, 16-byte aligned rows;
 * out may alias x and residual_out may alias residual. hidden % 8 == 0,
 * hidden <= 8192. weight: (hidden,) dtype.
 */
int sd_rmsnorm(const void* x, int64_t x_stride, const void* residual, int64_t residual_stride,
               const void* weight, void* out, int64_t out_stride, void* residual_out,
               int64_t residual_out_stride, int64_t rows, int32_t hidden, float eps,
               int32_t dtype, void* stream);

/*
 * Per-head q/k RMSNorm then rotate-half RoPE, in place: Qwen3Attention.forward
 * between the qkv projection and attention (nanovllm/models/qwen3.py:80-88)
 * with RotaryEmbedding.forward (layers/rotary_embedding.py:6-48).
 *   q: (num_tokens, num_q_heads, 128) by strides; k: (num_tokens, num_kv_heads, 128)
 *   (views into the qkv projection output work); q_weight / k_weight: (128,)
 *   dtype, NULL skips the norm (RoPE only).
 *   positions: (num_tokens,) int64; cos_sin: (max_position, cos_sin_stride)
 *   fp32 rows [cos(64) | sin(64)] — the reference's cos_sin_cache.
 * A token whose position is outside [0, max_position) is left unchanged.
 */
int sd_qk_norm_rope(void* q, int64_t q_stride_tok, int64_t q_stride_head, void* k,
                    int64_t k_stride_tok, int64_t k_stride_head, int64_t num_tokens,
                    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                    const void* q_weight, const void* k_weight, float eps,
                    const int64_t* positions, const float* cos_sin, int64_t cos_sin_stride,
                    int64_t max_position, int32_t dtype, void* stream);

/*
 * sd_qk_norm_rope followed by store_kvcache of the finished k rows and of v
 * (nanovllm/layers/attention.py:33-40), one launch: the draft step's q/k-norm,
 * RoPE and cache write (models/qwen3.py:80-88 then Attention.forward's store).
 * No counterpart entry in the reference, which runs them separately. Token t's
 * k and v rows go to slot slot_mapping[t] of the paged caches
 * (num_blocks, block_size, num_kv_heads, 128) with the given strides; slot -1
 * or outside the pool: not written. q, k, the caches: bit for bit what the two
 * separate calls leave. A token whose position has no cos/sin row stores its
 * k row unrotated, as it is left in place.
 */
int sd_qk_norm_rope_store(void* q, int64_t q_stride_tok, int64_t q_stride_head, void* k,
                          int64_t k_stride_tok, int64_t k_stride_head, const void* v,
                          int64_t v_stride_tok, int64_t v_stride_head, int64_t num_tokens,
                          int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                          const void* q_weight, const void* k_weight, float eps,
                          const int64_t* positions, const float* cos_sin,
                          int64_t cos_sin_stride, int64_t max_position, void* k_cache,
                          void* v_cache, int64_t cache_stride_block, int64_t cache_stride_pos,
                          int64_t cache_stride_head, int64_t num_blocks, int32_t block_size,
                          const int32_t* slot_mapping, int32_t dtype, void* stream);

/*
 * SiluAndMul (nanovllm/layers/activation.py:6-11): x (rows, 2*width) = [gate | up],
 * out (rows, width) = bf16(bf16(silu(gate)) * up). 16-byte aligned rows,
 * width % 8 == 0.
 */
int sd_silu_mul(const void* x, int64_t x_stride, void* out, int64_t out_stride, int64_t rows,
                int32_t width, int32_t dtype, void* stream);

/*
 * Sampler.forward (nanovllm/layers/sampler.py:6-12; the draft's per-step
 * sampling, spec_decode/draft_proposer.py:505-510): one token per row of
 * logits (rows, vocab), dtype bf16/f16/f32, into out_tokens (rows,) int64.
 *   temperatures == NULL, or a row's temperature <= 0: greedy argmax (first
 *   index among equal maxima, as torch.argmax).
 *   otherwise: argmax(softmax(l / T) / E), E ~ Exp(1), computed as
 *   argmax(l / T - log E) with E = max(-log U, 1e-10), U in (0, 1] from
 *   word (column % 4) of the Philox4x32-10 block keyed by rng_state[0] (seed)
 *   with counter (column / 4, row ^ high word of rng_state[1], low word of
 *   rng_state[1], 0).
 *   rng_state: (2,) int64 on the device, read only; the caller advances the
 *   offset between calls (on the stream, so graph replays advance it too).
 * Two launches: each row split over 4096-column workgroups, then a per-row
 * merge of their (key, column) partials held in the workspace
 * (sd_sample_workspace_size bytes, 8-byte aligned). rows <= 65535.
 */
size_t sd_sample_workspace_size(int64_t rows, int32_t vocab);
int sd_sample(const void* logits, int64_t logits_stride, int32_t dtype, int64_t rows,
              int32_t vocab, const float* temperatures, const int64_t* rng_state,
              int64_t* out_tokens, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Variable-length causal attention, the prefill branch of the attention layer:
 * flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
 * max_seqlen_k, softmax_scale, causal=True, block_table)
 * (nanovllm/layers/attention.py:64-70). Query row t of sequence b attends keys
 * [0, nk_b - nq_b + t] (bottom-right aligned), nq_b / nk_b from the cu arrays.
 *   q   : (total_q, num_q_heads, 128), row strides as given
 *   k/v : block_table == NULL: contiguous (total_k, num_kv_heads, 128) with
 *         kv_stride_tok / kv_stride_head (kv_stride_block unused), rows of
 *         sequence b from cu_seqlens_k[b];
 *         block_table != NULL: the paged cache, (num_blocks, block_size,
 *         num_kv_heads, 128) by kv_stride_block / kv_stride_tok /
 *         kv_stride_head (the prefix-cache case)
 *   out : (total_q, num_q_heads, 128)
 * head_dim 128, num_q_heads / num_kv_heads dividing 128, bf16/f16; 16-byte
 * aligned rows. One launch, no workspace.
 */
int sd_prefill_attention(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                         const void* k, const void* v, int64_t kv_stride_tok,
                         int64_t kv_stride_head, int64_t kv_stride_block, int64_t num_blocks,
                         int32_t block_size, const int32_t* block_table, int64_t bt_stride,
                         int32_t max_blocks_per_seq, const int32_t* cu_seqlens_q,
                         const int32_t* cu_seqlens_k, int32_t max_seqlen_q, int64_t total_q,
                         int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                         int32_t head_dim, float scale, int32_t dtype, void* out,
                         int64_t out_stride_tok, int64_t out_stride_head, void* stream);

/*
 * Workspace bytes of sd_verify_batch (0 for an empty batch).
 */
size_t sd_verify_batch_workspace_size(int64_t batch, int32_t k, int32_t vocab);

/*
 * Speculative verification by rejection sampling: `verify_batch`
 * (nanovllm/spec_decode/verify.py:39-183).
 *   draft   : (batch, k, vocab) by strides, bf16/f16/f32: the draft's raw logits
 *             (q_j = softmax(draft_j / T)), or its probabilities when
 *             draft_is_point_mass != 0 (the n-gram route; used as given)
 *   target  : (batch, k + 1, vocab) by strides: the target's logits
 *             (p_j = softmax(target_j / T))
 *   draft_tokens : (batch, k) int64, row stride tokens_stride_b
 *   temperatures : (batch,) fp32 or NULL (1); a temperature <= 0 is taken as 1
 *   rng_state    : (2,) int64 on the device: seed, offset (read only; the
 *                  caller advances the offset between calls)
 * Outputs: accepted (batch,) int64 = index of the first rejected candidate (k
 * when all pass; candidate j passes when u_j < min(1, p_j[x_j] / q_j[x_j]),
 * 0 when q_j[x_j] == 0); bonus (batch,) int64 drawn from
 * normalize(max(0, p_a - q_a)) at a = accepted with q_k = 0 (p_a when the
 * residual is all zero); accept_mask (batch, k) uint8 per-candidate tests.
 * u_j and the bonus race noise come from Philox4x32-10 (streams 1 and 2 of
 * the counter's last word; the bonus noise of column i is word i % 4 of the
 * block with counter (i / 4, ...)), so a call is a pure function of its inputs.
 * Three launches (row statistics, acceptance + residual race, merge); k <= 32.
 */
int sd_verify_batch(const void* draft, int64_t draft_stride_b, int64_t draft_stride_k,
                    int32_t draft_dtype, const void* target, int64_t target_stride_b,
                    int64_t target_stride_k, int32_t target_dtype, const int64_t* draft_tokens,
                    int64_t tokens_stride_b, const float* temperatures,
                    int32_t draft_is_point_mass, const int64_t* rng_state, int64_t batch,
                    int32_t k, int32_t vocab, int64_t* accepted, int64_t* bonus,
                    uint8_t* accept_mask, void* workspace, size_t workspace_bytes,
                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SPECDEC_AMD_H */
