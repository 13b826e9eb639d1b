/*
 * mce_abi.h -- C ABI of libmce.so, the gfx950 (MI355X) kernels behind the
 * `my_cuda_engine_cpp` op surface.
 *
 * Every entry point:
 *   - takes raw device pointers, element counts / strides (in elements) and a
 *     HIP stream handle passed as `void*` (a hipStream_t; NULL = legacy stream);
 *   - validates its arguments on the host and returns MCE_OK (0) or a nonzero
 *     MCE_ERR_* code, with a message available from mce_last_error();
 *   - launches asynchronously on `stream`: it never synchronises, never reads
 *     device memory on the host and never allocates device memory, so it may be
 *     recorded by hipStreamBeginCapture / torch.cuda.graph;
 *   - checks hipGetLastError() after its launches.
 *
 * dtype codes: MCE_F16 (IEEE half) and MCE_BF16 (bfloat16).  Index tensors are
 * int32, RoPE tables are fp32, as in the reference.
 *
 * Reference interfaces replaced (paths relative to the reference checkout):
 *   csrc/bindings.cpp:4-19,22-29   pybind op surface `my_cuda_engine_cpp`
 */
#ifndef MCE_ABI_H
#define MCE_ABI_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define MCE_API __attribute__((visibility("default")))
#else
#define MCE_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

enum {
  MCE_OK = 0,
  MCE_ERR_INVALID = 1,     /* bad pointer / shape / stride / value */
  MCE_ERR_UNSUPPORTED = 2, /* valid request this build has no kernel for */
  MCE_ERR_LAUNCH = 3,      /* the HIP runtime rejected a launch */
  MCE_ERR_WORKSPACE = 4    /* workspace missing or smaller than required */
};

enum { MCE_F16 = 0, MCE_BF16 = 1 };

/* Epilogues of mce_decode_gemm. */
enum { MCE_EPI_STORE = 0, MCE_EPI_ADD = 1, MCE_EPI_SWIGLU = 2 };

/* Message of the last failed call on this host thread ("" if none). */
MCE_API const char *mce_last_error(void);

/*
 * ABI version (major * 100 + minor) of the library; callers built against
 * this header should check mce_abi_version() == MCE_ABI_VERSION.
 * 101: mce_argmax_rows takes (workspace, workspace_bytes) before the stream.
 */
#define MCE_ABI_VERSION 101
MCE_API int mce_abi_version(void);

/*
 * Fused RMSNorm: out[r, :] = x[r, :] * rsqrt(mean(x[r, :]^2) + eps) * w, with
 * fp32 accumulation and one rounding to the storage type.
 * Replaces rmsnorm_cuda (csrc/kernels/rmsnorm.cu:110-130; binding
 * csrc/bindings.cpp:4-5,23).  Rows are `row_stride` elements apart; the last
 * dimension is contiguous.  Any hidden size >= 1 is accepted.
 */
MCE_API int mce_rmsnorm(int dtype, const void *input, const void *weight, void *output,
                int64_t rows, int64_t hidden, int64_t in_row_stride,
                int64_t out_row_stride, float eps, void *stream);

/*
 * Fused SwiGLU: out[t, j] = silu(gate_up[t, j]) * gate_up[t, I + j], j < I,
 * silu(x) = x / (1 + exp(-x)).  `inter` is I (half the input's last dim).
 * Replaces swiglu_cuda (csrc/kernels/swiglu.cu:29-52; binding
 * csrc/bindings.cpp:6,24).  Computes every row (the reference's guard at
 * swiglu.cu:13 writes only rows 0-1).
 */
MCE_API int mce_swiglu(int dtype, const void *gate_up, void *output, int64_t rows,
               int64_t inter, int64_t in_row_stride, int64_t out_row_stride,
               void *stream);

/*
 * Paged KV store: for each token n with s = slot_mapping[n] >= 0,
 *   key_cache[s / block_size, s % block_size, h, :]   = key[n, h, :]
 *   value_cache[s / block_size, s % block_size, h, :] = value[n, h, :]
 * Caches are contiguous [num_blocks, block_size, num_kv_heads, head_dim].
 * key/value rows are addressed n * *_stride_tok + h * *_stride_head (the last
 * dimension contiguous).  Slots >= num_blocks * block_size are skipped.
 * Replaces paged_kv_store_cuda (csrc/kernels/paged_kv.cu:45-69; binding
 * csrc/bindings.cpp:7,25), which hard-codes block_size 16 (paged_kv.cu:22).
 */
MCE_API int mce_paged_kv_store(int dtype, const void *key, const void *value,
                       void *key_cache, void *value_cache,
                       const int32_t *slot_mapping, int64_t num_tokens,
                       int num_kv_heads, int head_dim, int block_size,
                       int64_t num_blocks, int64_t key_stride_tok,
                       int64_t key_stride_head, int64_t value_stride_tok,
                       int64_t value_stride_head, void *stream);

/*
 * Workspace bytes mce_paged_attention_decode needs for these dimensions
 * (split-K partial softmax state).  Depends only on host-known sizes;
 * 0 means no workspace is needed (table capacities of at most 1024 tokens).
 */
MCE_API size_t mce_paged_attention_decode_workspace_size(int batch, int num_heads,
                                                 int num_kv_heads,
                                                 int max_blocks_per_seq,
                                                 int block_size);

/*
 * Paged decode attention (one query token per sequence), GQA:
 *   out[b, h, :] = sum_{t < ctx_b} softmax_t(scale * q[b,h] . k_t) v_t
 * with k_t/v_t at cache[block_tables[b, t / block_size], t % block_size,
 * h / (num_heads / num_kv_heads), :].  query/out are contiguous
 * [batch, num_heads, head_dim]; caches contiguous
 * [num_blocks, block_size, num_kv_heads, head_dim]; block_tables int32
 * [batch, max_blocks_per_seq]; context_lens int32 [batch].
 * Rows with ctx <= 0 are written as zeros.  ctx is clamped to
 * max_blocks_per_seq * block_size; block ids outside [0, num_blocks) are
 * clamped into range (the reference reads out of bounds there).
 * head_dim must be 128, block_size a power of two in [8, 256],
 * num_heads / num_kv_heads in [1, 8], num_blocks * block_size <= 2^32
 * token slots.
 * Workspace: 256-byte aligned, at least
 * mce_paged_attention_decode_workspace_size() bytes, no initialisation
 * needed; it is scratch for the duration of the call (two calls that run
 * concurrently need two workspaces).  It holds (J + batch) partial-state
 * slots of 520 bytes per query head, J ~ one workgroup per CU per group of
 * 8 kv heads (3.6 MB for 32 sequences x 24 heads on 256 CUs), whatever the
 * context lengths.
 * Replaces paged_attention_decode_cuda (csrc/kernels/flash_attn_paged.cu:
 * 144-168; binding csrc/bindings.cpp:8,26).
 */
MCE_API int mce_paged_attention_decode(int dtype, const void *query,
                               const void *key_cache, const void *value_cache,
                               const int32_t *block_tables,
                               const int32_t *context_lens, void *output,
                               int batch, int num_heads, int num_kv_heads,
                               int head_dim, int max_blocks_per_seq,
                               int block_size, int64_t num_blocks, float scale,
                               void *workspace, size_t workspace_bytes,
                               void *stream);

/*
 * mce_paged_attention_decode without the workspace argument: the split-K
 * partials go to a static scratch array of the library (file scope, 256-byte
 * aligned, MCE_DECODE_NOALLOC_SCRATCH_BYTES = 16 MiB, one copy per GPU the
 * library runs on, held until the process ends), so the call allocates
 * nothing.  Same arguments, results (bit for bit) and
 * validation otherwise.  Shapes whose workspace
 * (mce_paged_attention_decode_workspace_size) exceeds the scratch return
 * MCE_ERR_UNSUPPORTED.  Calls that overlap on one GPU share the scratch and
 * race: serialise them (one stream, or one call at a time).  The first call
 * on each device looks the scratch up with hipGetSymbolAddress; make it
 * outside stream capture.  No counterpart in the reference: for callers that
 * cannot allocate (code under HIP graph capture that must not touch the
 * allocator, tight serving loops, harnesses that forbid hipMalloc).
 */
#define MCE_DECODE_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)

MCE_API int mce_paged_attention_decode_noalloc(int dtype, const void *query,
                                       const void *key_cache, const void *value_cache,
                                       const int32_t *block_tables,
                                       const int32_t *context_lens, void *output,
                                       int batch, int num_heads, int num_kv_heads,
                                       int head_dim, int max_blocks_per_seq,
                                       int block_size, int64_t num_blocks, float scale,
                                       void *stream);

/*
 * One decode token per sequence with the rotary embedding and the paged
 * store of the new token fused in: rotates query[b] and key[b] at
 * positions[b] (rows of cos/sin_table as in mce_rope_inplace; positions
 * outside [0, table_rows) are not rotated), writes the rotated key and value
 * to the page slot slot_mapping[b] (skipped when outside the pool), then
 * computes mce_paged_attention_decode with the rotated query.  Outputs and
 * caches are bit-identical to mce_rope_kv_store (query_out given) followed by
 * mce_paged_attention_decode.  query/key/value are [batch, heads, head_dim]
 * rows q_stride / kv_stride elements apart (views into one fused projection
 * output).  Only for table capacities (max_blocks_per_seq * block_size) of
 * at most 1024 tokens, the per-sequence mode; larger ones return
 * MCE_ERR_UNSUPPORTED.  No workspace.  No single counterpart in the
 * reference: it fuses the three calls of its decode step
 * (engine/models/llama.py:117-134: rope_inplace, paged_kv_store,
 * paged_attention_decode).
 */
MCE_API int mce_paged_attention_decode_rope(int dtype, const void *query, const void *key,
                                    const void *value, void *key_cache, void *value_cache,
                                    const float *cos_table, const float *sin_table,
                                    const int32_t *positions, const int32_t *slot_mapping,
                                    const int32_t *block_tables, const int32_t *context_lens,
                                    void *output, int batch, int num_heads, int num_kv_heads,
                                    int head_dim, int max_blocks_per_seq, int block_size,
                                    int64_t num_blocks, int64_t table_rows, int64_t q_stride,
                                    int64_t kv_stride, float scale, void *stream);

/*
 * In-place rotary embedding (half-split / rotate_half form), i < head_dim/2:
 *   (x_i, x_{i+D/2}) <- (x_i c - x_{i+D/2} s, x_i s + x_{i+D/2} c),
 *   c = cos_table[pos, i], s = sin_table[pos, i], pos = positions[token].
 * query is [batch, seq, num_heads, head_dim], key [batch, seq, num_kv_heads,
 * head_dim] (key may be NULL), both with arbitrary strides except a
 * contiguous last dimension; positions int32 [batch * seq] (contiguous);
 * tables fp32 [table_rows, head_dim / 2] contiguous.  Tokens whose position
 * is outside [0, table_rows) are left unrotated.
 * Replaces rope_inplace_cuda (csrc/kernels/rope.cu:64-99; binding
 * csrc/bindings.cpp:9-13,27).
 */
MCE_API int mce_rope_inplace(int dtype, void *query, void *key, const float *cos_table,
                     const float *sin_table, const int32_t *positions,
                     int batch, int seq_len, int num_heads, int num_kv_heads,
                     int head_dim, int64_t table_rows, int64_t q_stride_b,
                     int64_t q_stride_s, int64_t q_stride_h,
                     int64_t k_stride_b, int64_t k_stride_s,
                     int64_t k_stride_h, void *stream);

/*
 * RoPE of query and key in place, then the paged store of the rotated key and
 * of value: the same result, bit for bit, as mce_rope_inplace (batch =
 * num_tokens, seq_len = 1) followed by mce_paged_kv_store on the same tokens,
 * in one launch.  With query_out non-null the rotated query goes to the
 * contiguous rows query_out[num_tokens, num_heads, head_dim] instead (query
 * untouched), ready for mce_paged_attention_decode.  Tokens are flat: positions[t] and slot_mapping[t] per
 * token; query/key/value rows are addressed by (token, head) strides in
 * elements.  No single counterpart in the reference: it fuses the two calls
 * its decode step makes back to back (engine/models/llama.py:117-127 calls
 * rope_inplace, then paged_kv_store), for the engine's decode and prefill.
 */
MCE_API int mce_rope_kv_store(int dtype, void *query, void *query_out, void *key,
                      const void *value,
                      void *key_cache, void *value_cache, const float *cos_table,
                      const float *sin_table, const int32_t *positions,
                      const int32_t *slot_mapping, int64_t num_tokens, int num_heads,
                      int num_kv_heads, int head_dim, int64_t table_rows, int block_size,
                      int64_t num_blocks, int64_t q_stride_tok, int64_t q_stride_head,
                      int64_t k_stride_tok, int64_t k_stride_head, int64_t v_stride_tok,
                      int64_t v_stride_head, void *stream);

/*
 * Decode-sized projection: out[m, :n] (op)= x[m, :k] . w[:n, :k]^T for m <= 16
 * rows (one token per sequence), w row-major [n, k] (the Hugging Face
 * [out_features, in_features] layout), fp32 accumulation:
 *   MCE_EPI_STORE  out = x w^T
 *   MCE_EPI_ADD    out += x w^T            (in-place residual add)
 *   MCE_EPI_SWIGLU w is [2n, k] (gate rows, then up rows);
 *                  out[:, j] = silu(x w_gate_j) * (x w_up_j)
 * x rows x_stride elements apart, out rows out_stride apart (out must not
 * overlap x).  Needs dtype MCE_F16 (the engine's weights are fp16),
 * n % 16 == 0 and k in {2048, 3072, 4096}, or k == 8192 for m <= 8 without
 * SwiGLU; other dtypes and shapes return MCE_ERR_UNSUPPORTED (callers then
 * use a library GEMM).
 * No single counterpart in the reference: its decode step runs these
 * projections through torch.matmul, then a separate SwiGLU kernel and
 * residual adds (engine/models/llama.py:94-110,143-165,174).
 */
MCE_API int mce_decode_gemm(int dtype, const void *x, const void *w, void *out, int m, int n,
                    int k, int64_t x_stride, int64_t out_stride, int epilogue, void *stream);

/*
 * RMSNorm fused in front of mce_decode_gemm: out (op)= rmsnorm(x) w^T with
 * rmsnorm(x)[m, :] = x[m, :] / sqrt(mean(x[m, :]^2) + eps) * norm_weight
 * (norm_weight [k]), the normalised rows bit-identical to mce_rmsnorm's
 * output; same epilogues, layouts and shape rules as mce_decode_gemm, k in
 * {2048, 3072, 4096}.  The normalised rows are not written out.  Replaces the
 * RMSNorm + projection pairs of the reference decode step
 * (engine/models/llama.py:82-108 input_layernorm + q/k/v, :147-159
 * post_attention_layernorm + gate/up, :169-174 final norm + lm_head; with
 * csrc/kernels/rmsnorm.cu:35-130).
 */
MCE_API int mce_rmsnorm_decode_gemm(int dtype, const void *x, const void *norm_weight, float eps,
                                    const void *w, void *out, int m, int n, int k,
                                    int64_t x_stride, int64_t out_stride, int epilogue,
                                    void *stream);

/*
 * Greedy token of each logits row: out[r] = index of the largest value of
 * logits[r, 0:cols] (rows row_stride elements apart; NaN ranks above every
 * number and the lower index wins among equals, as torch.argmax does).
 * Replaces the host-side torch.argmax between replays of the reference's
 * decode loop (benchmarks/benchmark_engine.py:255-265), so the next input
 * ids stay on the device inside a captured graph.  16-byte aligned rows with a
 * row stride that is a multiple of 8 are split over up to 64 workgroups each
 * (4096 columns per part), whose partial maxima go through `workspace` (8-byte
 * aligned, mce_argmax_rows_workspace_size() bytes, no initialisation; calls
 * that run concurrently need separate workspaces) to a second, reducing
 * launch; other rows take one workgroup each and no workspace (NULL allowed).
 */
/* Workspace bytes mce_argmax_rows needs: rows x parts x 8 (0 for an empty batch). */
MCE_API size_t mce_argmax_rows_workspace_size(int64_t rows, int64_t cols);

MCE_API int mce_argmax_rows(int dtype, const void *logits, int64_t rows, int64_t cols,
                            int64_t row_stride, int64_t *out, void *workspace,
                            size_t workspace_bytes, void *stream);

/*
 * Prepares the next decode step on the device (one launch, capturable):
 * when token_log is non-null, token_log[step * batch + b] = input_ids[b] for
 * step = *step_counter (skipped past log_capacity rows) and *step_counter is
 * incremented; then for every sequence b: positions[b] += 1,
 * context_lens[b] += 1 and slot_mapping[b] = block_tables[b][p / block_size]
 * * block_size + p % block_size for the new position p (-1 when p falls
 * outside the max_blocks_per_seq-wide, zero-padded int32 table).  Replaces
 * the host-side preparation of every replay in the reference
 * (engine/runner.py:39-60 _prepare_inputs, :153-178 execute; slot rule of
 * engine/cache.py:48-57).
 */
MCE_API int mce_decode_advance(const int32_t *block_tables, int32_t *positions,
                               int32_t *context_lens, int32_t *slot_mapping,
                               const int64_t *input_ids, int64_t *token_log,
                               int32_t *step_counter, int batch, int max_blocks_per_seq,
                               int block_size, int log_capacity, void *stream);

/*
 * Causal prefill attention over contiguous Q/K/V, GQA:
 *   out[b, s, h, :] = sum_{t <= s} softmax_t(scale * q[b,s,h] . k[b,t,g]) v[b,t,g]
 * with g = h / (num_heads / num_kv_heads).  query/out contiguous
 * [batch, seq, num_heads, head_dim]; key/value contiguous
 * [batch, seq, num_kv_heads, head_dim].  head_dim must be 128.
 * Replaces prefill_attention_cuda (csrc/kernels/prefill_attention.cu:271-309;
 * binding csrc/bindings.cpp:14-19,28).
 */
MCE_API int mce_prefill_attention(int dtype, const void *query, const void *key,
                          const void *value, void *output, int batch,
                          int seq_len, int num_heads, int num_kv_heads,
                          int head_dim, float scale, void *stream);

/*
 * Chunked causal prefill attention with K/V from the page pool: query
 * [batch, seq_len, num_heads, 128] holds the last seq_len positions of each
 * sequence; sequence b has context_lens[b] tokens (clamped into [seq_len,
 * max_blocks_per_seq * block_size]) whose K/V rows are in key_cache /
 * value_cache [num_blocks, block_size, num_kv_heads, 128] at the slots of
 * block_tables[b] (int32 [batch, max_blocks_per_seq], block ids clamped into
 * the pool).  Query i of sequence b is position context_lens[b] - seq_len + i
 * and attends causally to keys 0 .. that position; output like query.  The
 * pool must be smaller than 2 GiB, max_blocks_per_seq <= 8192.  With
 * context_lens == seq_len and an identity table it equals
 * mce_prefill_attention on the same K/V bit for bit.  Widens the reference's
 * prefill (benchmarks/benchmark_engine.py:64-89 with
 * csrc/kernels/prefill_attention.cu:271-309: contiguous K/V of the whole
 * prompt) to prompts processed in chunks against the cached prefix.
 * Key split (optional): on small grids (batch * num_kv_heads *
 * ceil(seq_len * G / 128) at most half the CUs: short chunks of few
 * sequences) a non-null workspace of mce_prefill_attention_paged_workspace_size()
 * bytes, 256-byte aligned (MCE_ERR_WORKSPACE otherwise; no initialisation;
 * calls sharing one race), lets every query block whose keys span at least
 * 1024 positions be cut into parts of at least 512 keys on separate
 * workgroups, merged by a second launch.  It pays off behind long cached
 * prefixes (the second launch costs a few microseconds even when no block is
 * cut); with workspace == NULL, or on larger grids, the keys are not split.
 */
/* Workspace bytes mce_prefill_attention_paged needs for this shape (0: none). */
MCE_API size_t mce_prefill_attention_paged_workspace_size(int batch, int seq_len, int num_heads,
                                                          int num_kv_heads);

MCE_API int mce_prefill_attention_paged(int dtype, const void *query, const void *key_cache,
                                        const void *value_cache, const int32_t *block_tables,
                                        const int32_t *context_lens, void *output, int batch,
                                        int seq_len, int num_heads, int num_kv_heads,
                                        int head_dim, int max_blocks_per_seq, int block_size,
                                        int64_t num_blocks, float scale, void *workspace,
                                        size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MCE_ABI_H */
