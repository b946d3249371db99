/*
 * edgerag_amd.h -- C ABI of the MI355X (gfx950) ragged decoder-step library.
 *
 * One shared library, libedgerag_amd.so, exports every entry point below. They take raw device
 * pointers, explicit sizes and strides, and a hipStream_t passed as void*. No torch types cross
 * this boundary, so any host language with a C FFI can bind it (ctypes, cgo, JNI, N-API).
 *
 * Conventions shared by every entry point:
 *   - return 0 on success, a positive EDGERAG_E* code on failure; edgerag_last_error() then holds
 *     a thread-local, human-readable message;
 *   - nothing here allocates device memory or synchronises the stream: callers own every buffer,
 *     including the attention workspace sized by edgerag_attn_plan();
 *   - kernels are enqueued on `stream` and run asynchronously; the entry points are reentrant and
 *     keep no mutable global state, so calls from different host threads on different streams do
 *     not interact -- except edgerag_paged_attention_noalloc, whose calls share one static
 *     per-GPU scratch array (see there);
 *   - element types are EDGERAG_F32 / EDGERAG_F16 / EDGERAG_BF16 (see below).
 *
 * The reference (Tejas544/edgerag) is pure Python/PyTorch and has no FFI; each declaration cites
 * the Python seam it replaces (file:line in the reference checkout).
 */
#ifndef EDGERAG_AMD_H
#define EDGERAG_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------------------------- */
#define EDGERAG_OK 0
#define EDGERAG_EINVAL 1        /* bad argument: null pointer, shape, dtype or range */
#define EDGERAG_EHIP 2          /* the HIP runtime reported an error (launch, copy) */
#define EDGERAG_EWORKSPACE 3    /* workspace or plan buffer smaller than required */
#define EDGERAG_EUNSUPPORTED 4  /* valid request this build does not implement */

/* ---- parts of a paged-attention launch (edgerag_paged_attention) ------------------------- */
#define EDGERAG_ATTN_TILES 1
#define EDGERAG_ATTN_ROWS 2
#define EDGERAG_ATTN_COMBINE 4
#define EDGERAG_ATTN_ALL 7
#define EDGERAG_ATTN_TILES_SHARED 8 /* modifier of EDGERAG_ATTN_TILES, see below */

/* ---- element types ----------------------------------------------------------------------- */
#define EDGERAG_F32 0
#define EDGERAG_F16 1
#define EDGERAG_BF16 2

/* Message describing the last failure on the calling thread ("" if none). */
const char* edgerag_last_error(void);

/* Library version string, e.g. "edgerag_amd 0.1.0 gfx950". */
const char* edgerag_version(void);

/* ==== KV cache: slot-mapped append, gather, block copy ====================================== */

/*
 * Slot-mapped KV append: for every token t with slot s = slot_mapping[t] >= 0,
 *   key_pool  [h, s / block_size, s % block_size, :] = key  [t, h, :]
 *   value_pool[h, s / block_size, s % block_size, :] = value[t, h, :]
 * for h in [0, n_kv_heads). Pools are head-major [n_kv_heads, num_blocks, block_size, head_dim]
 * and contiguous. Source element (t, h, x) lives at src + t*stride_tok + h*stride_head + x (in
 * elements; the head_dim axis is contiguous). Conversion src_dtype -> pool_dtype rounds to
 * nearest-even, exactly like torch's Tensor.to(). Slots < 0 are skipped (padding); slots at or
 * beyond num_blocks*block_size are skipped too, so a bad slot can never write out of bounds.
 * Either of key/value may be NULL (with its pool) to append only the other.
 *
 * Replaces PagedKVCache._write, edgerag/cache/paged.py:186-206, with the slot mapping
 * slot = table[pos // block_size] * block_size + pos % block_size built once per step.
 */
int edgerag_kv_append(const void* key, const void* value, int32_t src_dtype,
                      int64_t src_stride_tok, int64_t src_stride_head,
                      const int32_t* slot_mapping, int32_t num_tokens,
                      void* key_pool, void* value_pool, int32_t pool_dtype,
                      int32_t n_kv_heads, int32_t num_blocks, int32_t block_size,
                      int32_t head_dim, void* stream);

/*
 * Materialise one sequence's history: out[h, p, :] = pool[h, block_ids[p / bs], p % bs, :] for
 * p < seq_len, out contiguous [n_kv_heads, seq_len, head_dim] in the pool's dtype. Block ids
 * outside [0, num_blocks) produce zeros rather than an out-of-bounds read.
 *
 * Replaces PagedKVCache.gather/_gather_pool, edgerag/cache/paged.py:208-238 (including the
 * [:seq_len] slice that keeps the final block's slack out of attention).
 */
int edgerag_kv_gather(const void* pool, int32_t dtype, int32_t n_kv_heads, int32_t num_blocks,
                      int32_t block_size, int32_t head_dim, const int32_t* block_ids,
                      int32_t seq_len, void* out, void* stream);

/*
 * Copy whole blocks inside one pool: pool[:, dst[i]] = pool[:, src[i]] for i < n_pairs, every
 * head. Pairs must not overlap (no block is both a source and a destination). Ids outside
 * [0, num_blocks) are skipped.
 *
 * Replaces the copy-on-write content copy of PagedKVCache._unshare_write_range,
 * edgerag/cache/paged.py:179-182 (and the pool[:, blocks] copies of cache/preemption.py:125-126).
 */
int edgerag_kv_copy_blocks(void* pool, int32_t dtype, int32_t n_kv_heads, int32_t num_blocks,
                           int32_t block_size, int32_t head_dim, const int32_t* src_blocks,
                           const int32_t* dst_blocks, int32_t n_pairs, void* stream);

/* ==== Ragged paged attention =============================================================== */

/*
 * Host-only planning for edgerag_paged_attention (no GPU call is made).
 *
 * The batch holds num_reqs requests packed token-major. Request r owns query tokens
 * [query_start_loc[r], query_start_loc[r+1]) (c_r of them) and, after this step's append,
 * context_lens[r] = L_r visible tokens. Query i of request r sits at logical position
 * L_r - c_r + i and attends keys [0, L_r - c_r + i] -- causal within the chunk, full over the
 * cached prefix. c_r = 1 is a decode; c_r = 0 contributes nothing.
 *
 * Writes the work list into plan[0 .. *plan_words) (int32 words; upload it to the device as-is)
 * and the device workspace size the run needs into *workspace_bytes. With plan == NULL only the
 * two sizes are computed. Fails with EDGERAG_EINVAL if c_r > L_r, L_r needs more than
 * max_blocks_per_seq blocks, or the shape is unsupported, and with EDGERAG_EWORKSPACE if
 * plan_capacity_words is too small.
 *
 * Together with edgerag_paged_attention this replaces, per request, build_causal_mask +
 * sdpa_attention over PagedKVCache.gather (edgerag/core/layers.py:137-167, :227-254;
 * edgerag/cache/paged.py:208-238) and, for c_r = 1, paged_attention_reference /
 * fused_paged_attention (edgerag/cache/fused.py:89-167, :242-286).
 */
int edgerag_attn_plan(const int32_t* query_start_loc, const int32_t* context_lens,
                      int32_t num_reqs, int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                      int32_t block_size, int32_t max_blocks_per_seq, int32_t dtype,
                      int32_t* plan, int64_t plan_capacity_words, int64_t* plan_words,
                      int64_t* workspace_bytes);

/*
 * edgerag_attn_plan with planning flags. Decode rows (requests with c * n_q_heads / n_kv_heads
 * <= 8 query vectors) are by default planned as one workgroup per (request, kv head) whose waves
 * split the context and merge in LDS (no split partials, no merge launch), whenever the fast
 * decode kernel takes the shape, every such context fits 16 waves of 64 blocks and those
 * workgroups make at most one round over the CUs (two when no context passes 1,536 tokens);
 * otherwise, or with EDGERAG_PLAN_SPLIT_ROWS, as one workgroup per KV split merged through fp32
 * partials in the workspace. Results agree to fp32 rounding either way. A batch with fewer such
 * workgroups than CUs (few decodes) instead cuts every row context into parts of 8 waves, one
 * workgroup each, whose partials sit in S fixed slots per (token, query head): plan word 21
 * holds S (0 when the rows are not slotted), and every row token then has a merge row.
 *
 * A batch with both prefill tiles and decode rows is planned for one of two runs, recorded in
 * plan word 20 (1: two streams, 0: one): the tiles (EDGERAG_ATTN_TILES | EDGERAG_ATTN_TILES_SHARED)
 * on one stream beside the rows (EDGERAG_ATTN_ROWS) on another, joined before
 * EDGERAG_ATTN_COMBINE; or EDGERAG_ATTN_ALL on one stream. The planner picks two streams when the
 * tiles fill every CU at one workgroup each and the rows read at least 256 MiB of K/V;
 * EDGERAG_PLAN_OVERLAP asks for it whenever the batch holds both. Either run of either plan gives
 * the same results; the plan only sizes the work items for the run it names.
 */
#define EDGERAG_PLAN_SPLIT_ROWS 1
#define EDGERAG_PLAN_OVERLAP 2
int edgerag_attn_plan_ex(const int32_t* query_start_loc, const int32_t* context_lens,
                         int32_t num_reqs, int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                         int32_t block_size, int32_t max_blocks_per_seq, int32_t dtype,
                         int32_t flags, int32_t* plan, int64_t plan_capacity_words,
                         int64_t* plan_words, int64_t* workspace_bytes);

/*
 * Run the planned attention. plan_host is the plan edgerag_attn_plan wrote (read on the host for
 * the launch configuration) and plan_dev its device copy (read by the kernels). q:
 * [num_tokens, n_q_heads, head_dim] at q + t*q_stride_tok + h*q_stride_head; out likewise. Pools
 * are head-major and contiguous; block_tables is [num_reqs, block_tables_stride] int32 on the
 * device; query_start_loc and context_lens are the device copies of the arrays given to
 * edgerag_attn_plan. scale multiplies q.k (1/sqrt(head_dim) in the reference). Query head h reads
 * kv head h / (n_q_heads / n_kv_heads) (repeat_interleave order, layers.py:117-134).
 * Accumulation is fp32; out is written in `dtype` (the dtype of q and the pools). A query row with
 * no visible key is written as zeros, never NaN. Block ids outside [0, num_blocks) contribute
 * nothing. workspace must hold the *workspace_bytes the plan reported (NULL if that is 0).
 *
 * parts selects what is enqueued, so a caller can overlap the two kinds of work on two streams:
 *   EDGERAG_ATTN_TILES    prefill query tiles (MFMA-bound);
 *   EDGERAG_ATTN_ROWS     decode rows (HBM-bound);
 *   EDGERAG_ATTN_COMBINE  the merge of split partials (of tiles and of rows alike), which must be
 *                         enqueued after both of the other parts have completed;
 *   EDGERAG_ATTN_ALL      all three in order on `stream`.
 * Tiles and rows write disjoint outputs and partials. EDGERAG_ATTN_TILES_SHARED, added to
 * EDGERAG_ATTN_TILES, runs the MFMA tiles at one workgroup per CU, which leaves the rest of every
 * CU's registers to decode rows enqueued on another stream; enqueue the tiles first. It changes
 * nothing in the results.
 */
int edgerag_paged_attention(const int32_t* plan_host, const int32_t* plan_dev, int64_t plan_words,
                            const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                            const void* key_pool, const void* value_pool, int32_t dtype,
                            const int32_t* block_tables, int64_t block_tables_stride,
                            const int32_t* query_start_loc, const int32_t* context_lens,
                            int32_t num_reqs, int32_t num_tokens, int32_t n_q_heads,
                            int32_t n_kv_heads, int32_t head_dim, int32_t block_size,
                            int32_t num_blocks, float scale,
                            void* out, int64_t out_stride_tok, int64_t out_stride_head,
                            void* workspace, int64_t workspace_bytes, int32_t parts,
                            void* stream);

/*
 * The decode step's KV append and its attention in one call: exactly edgerag_kv_append(new_key,
 * new_value, new_dtype, new_stride_tok, new_stride_head, slot_mapping, num_tokens, key_pool,
 * value_pool, dtype, ...) followed by edgerag_paged_attention(..., EDGERAG_ATTN_ALL), with the
 * same results. When every work item of the plan is a decode row on the fast decode kernel (the
 * usual decode batch) and the new rows are in the pool dtype and 16-byte aligned, it is one
 * launch: the waves that reach a request's new positions read them from new_key / new_value and
 * write them to the pools at their slots; the attention treats a token's new K/V as sitting at
 * its position in the block table, as slot_mapping does when built from the tables. Otherwise
 * (prefill tiles in the batch, other layouts) it enqueues the two launches.
 *
 * Replaces PagedKVCache._write followed by fused_paged_attention for a decode step
 * (edgerag/cache/paged.py:186-206; edgerag/cache/fused.py:242-286).
 */
int edgerag_paged_attention_append(
    const void* new_key, const void* new_value, int32_t new_dtype, int64_t new_stride_tok,
    int64_t new_stride_head, const int32_t* slot_mapping, const int32_t* plan_host,
    const int32_t* plan_dev, int64_t plan_words, const void* q, int64_t q_stride_tok,
    int64_t q_stride_head, void* key_pool, void* value_pool, int32_t dtype,
    const int32_t* block_tables, int64_t block_tables_stride, const int32_t* query_start_loc,
    const int32_t* context_lens, int32_t num_reqs, int32_t num_tokens, int32_t n_q_heads,
    int32_t n_kv_heads, int32_t head_dim, int32_t block_size, int32_t num_blocks, float scale,
    void* out, int64_t out_stride_tok, int64_t out_stride_head, void* workspace,
    int64_t workspace_bytes, void* stream);

/*
 * Fixed-capacity form of edgerag_paged_attention for decode-only batches, for HIP graph capture.
 * The launch configuration depends only on the capacities, never on the plan: max_row_items
 * waves run the decode-row kernel and max_combine_rows x ceil(n_q_heads/4) the split merge, and
 * every wave reads its item (or returns) from the plan in device memory. A caller can therefore
 * capture this call once and, before each replay, rewrite plan_dev, query_start_loc,
 * context_lens and block_tables in place with a new edgerag_attn_plan output, provided that plan
 * has no prefill tiles (every request has c * n_q_heads / n_kv_heads <= 8 query vectors), at most
 * max_row_items items, at most max_combine_rows combine rows, at most max_partials split
 * partials and no request with more than max_row_vecs query vectors. The workspace holds
 * max_partials partials: (m, l) pairs at offset 0, accumulators at round_up(8 * max_partials,
 * 256); size it with that formula. Semantics are those of edgerag_paged_attention.
 * row_waves > 0 runs workgroup-split rows instead (one workgroup of row_waves waves per row item,
 * merged in LDS; plans whose word 19, the row-wave count, is nonzero, i.e. planned without
 * EDGERAG_PLAN_SPLIT_ROWS). Such a plan may still cut a context into parts (one row item each,
 * merged by the combine launch through partials: batches of few decodes); pass
 * max_combine_rows = 0 only for plans without combine rows (word 16 zero), which then need no
 * workspace. slots: the plan's word 21. With slots > 0 (parts in fixed slots, row_waves > 0) the
 * merge launch addresses every partial from its thread index, reads the token count from the
 * plan and takes one round trip; max_combine_rows is then the token capacity and max_partials
 * must hold max_combine_rows * n_q_heads * slots partials. A replayed plan whose word 21 differs
 * from `slots` gets NaN outputs instead of a wrong merge.
 *
 * No counterpart in the reference: it exists so that the decode step of the serving loop
 * (edgerag/serve/executor.py:138-154 replaced by one packed forward) can be replayed from a graph.
 */
/* Upper bound on the row items of any decode-only plan with a nonzero row-wave count that
 * edgerag_attn_plan makes for at most max_reqs requests of contexts up to max_context tokens:
 * the max_row_items to pass edgerag_paged_attention_fixed with row_waves > 0. -1 for bad
 * arguments. */
int64_t edgerag_attn_fixed_row_items(int32_t max_reqs, int32_t n_kv_heads, int32_t max_context,
                                     int32_t block_size);
int edgerag_paged_attention_fixed(const int32_t* plan_dev, int32_t max_row_items,
                                  int32_t max_combine_rows, int32_t max_row_vecs,
                                  int64_t max_partials, int32_t row_waves, int32_t slots,
                                  const void* q, int64_t q_stride_tok,
                                  int64_t q_stride_head, const void* key_pool,
                                  const void* value_pool, int32_t dtype,
                                  const int32_t* block_tables, int64_t block_tables_stride,
                                  const int32_t* query_start_loc, const int32_t* context_lens,
                                  int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                                  int32_t block_size, int32_t num_blocks, float scale,
                                  void* out, int64_t out_stride_tok, int64_t out_stride_head,
                                  void* workspace, int64_t workspace_bytes, void* stream);

/*
 * edgerag_paged_attention without a workspace argument: the same plan, arguments, parts mask and
 * results (bit for bit), with the split partials kept in a static device array of
 * EDGERAG_ATTN_SCRATCH_BYTES that the library holds on each GPU it runs on until the process
 * ends. It calls no hipMalloc / hipFree and no allocating routine. The first call on a device
 * looks the array's address up (hipGetSymbolAddress) with that device current; the stream must
 * belong to the current device. A plan whose partials need more than EDGERAG_ATTN_SCRATCH_BYTES
 * (edgerag_attn_plan's *workspace_bytes) is refused with EDGERAG_EWORKSPACE before anything is
 * enqueued. Every call on one GPU shares that GPU's array: calls that overlap in time on one GPU
 * (other streams, other host threads) race on it and must be ordered by the caller; the parts of
 * one step split over two streams (EDGERAG_ATTN_TILES / _ROWS, then _COMBINE) write disjoint
 * partials and are one call in this sense. Partials are written before they are read in every
 * call, so the array's leftover contents never matter.
 *
 * No counterpart in the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 */
#define EDGERAG_ATTN_SCRATCH_BYTES (32 * 1024 * 1024)
int edgerag_paged_attention_noalloc(const int32_t* plan_host, const int32_t* plan_dev,
                                    int64_t plan_words, const void* q, int64_t q_stride_tok,
                                    int64_t q_stride_head, const void* key_pool,
                                    const void* value_pool, int32_t dtype,
                                    const int32_t* block_tables, int64_t block_tables_stride,
                                    const int32_t* query_start_loc, const int32_t* context_lens,
                                    int32_t num_reqs, int32_t num_tokens, int32_t n_q_heads,
                                    int32_t n_kv_heads, int32_t head_dim, int32_t block_size,
                                    int32_t num_blocks, float scale, void* out,
                                    int64_t out_stride_tok, int64_t out_stride_head,
                                    int32_t parts, void* stream);

/* ==== Weight-only INT8 / INT4 quantisation and linear ===================================== */

/*
 * Group-wise symmetric quantisation of weight [N, K] (row-major, `w_dtype`) along K:
 *   amax = max |w| over each group of group_size; scale = amax / qmax (fp32, or 1.0 if amax == 0)
 *   code = clamp(round_half_even(w / scale), -qmax, qmax), qmax = 7 (bits 4) or 127 (bits 8)
 * packed: bits 8 -> [N, K] uint8 two's complement; bits 4 -> [N, K/2] uint8 with byte j holding
 * (code[2j] + 8) | (code[2j+1] + 8) << 4. scales: [N, K/group_size] fp16 (rounded from fp32).
 * Bit-identical to the reference. K % group_size must be 0 (and K even for bits 4).
 *
 * Replaces quantize_groupwise + pack_int4 (edgerag/core/quant.py:60-95, :110-125) as called by
 * QuantLinear.load_weight (edgerag/core/linear.py:166-184).
 */
int edgerag_quantize(const void* weight, int32_t w_dtype, int32_t n, int32_t k, int32_t bits,
                     int32_t group_size, uint8_t* packed, void* scales_f16, void* stream);

/*
 * Reconstruct the fp16 weight [N, K]: w = fp16(code) * scale, product rounded to fp16.
 *
 * Replaces QuantLinear.dequantized (edgerag/core/linear.py:186-192 -> unpack_int4,
 * dequantize_groupwise, edgerag/core/quant.py:98-138).
 */
int edgerag_dequantize(const uint8_t* packed, const void* scales_f16, int32_t n, int32_t k,
                       int32_t bits, int32_t group_size, void* weight_f16, void* stream);

/*
 * y[M, N] = x[M, K] . W^T (+ bias), W = fp16(code * scale) exactly as edgerag_dequantize builds
 * it, fp32 accumulation, y rounded to x's dtype. x: row stride x_stride (elements), contiguous
 * along K; y: row stride y_stride. x/y dtype: EDGERAG_F16 (all M) or EDGERAG_F32 (correctness
 * path). bias: [N] fp16 or NULL. M = 0 is a no-op.
 *
 * Replaces QuantLinear.forward = F.linear(x, dequantized().to(x.dtype), bias)
 * (edgerag/core/linear.py:194-196) without materialising the fp16 weight: packed weights are
 * streamed from HBM once and dequantised in registers.
 */
int edgerag_quant_linear(const void* x, int32_t x_dtype, int64_t x_stride, int32_t m, int32_t k,
                         const uint8_t* packed, const void* scales_f16, const void* bias_f16,
                         int32_t n, int32_t bits, int32_t group_size, void* y, int64_t y_stride,
                         void* stream);

/*
 * edgerag_quant_linear with a workspace, for the shapes where the tiled GEMM beats the streaming
 * GEMV (decode batches of 17..64 tokens on large layers, 40..64 tokens on most) or where the tiled
 * GEMM's output tiles would not fill the GPU (larger M on narrow layers). There the 64x64-tile
 * GEMM runs, with K cut into 2..16 equal ranges when a cost model says the GPU needs them: one
 * launch writes each range's fp32 partial tiles to the workspace, a second adds them in range
 * order and writes y (the same bits on every run). Results equal edgerag_quant_linear's to the
 * linear tolerance (the fp32 sums are ordered differently), not bit for bit.
 *
 * workspace: 16-byte aligned, at least edgerag_quant_linear_workspace_bytes(M, K, N, bits,
 * group_size) bytes, any contents. Launches that share a workspace must be ordered (one stream).
 * With a smaller, unaligned or NULL workspace, a shape that does not split K still takes the tiled
 * GEMM when the route says so; one that would split runs edgerag_quant_linear.
 *
 * Replaces QuantLinear.forward (edgerag/core/linear.py:194-196), as edgerag_quant_linear does.
 */
int edgerag_quant_linear_ws(const void* x, int32_t x_dtype, int64_t x_stride, int32_t m, int32_t k,
                            const uint8_t* packed, const void* scales_f16, const void* bias_f16,
                            int32_t n, int32_t bits, int32_t group_size, void* y, int64_t y_stride,
                            void* workspace, int64_t workspace_bytes, void* stream);
/* Workspace bytes edgerag_quant_linear_ws uses for this shape: 0 when it does not split K, and
 * never more than EDGERAG_QUANT_WORKSPACE_MAX. */
int64_t edgerag_quant_linear_workspace_bytes(int32_t m, int32_t k, int32_t n, int32_t bits,
                                             int32_t group_size);
#define EDGERAG_QUANT_WORKSPACE_MAX (8 * 1024 * 1024)

/*
 * SwiGLU through one launch: W = [gate; up] is the packed INT8 per-channel weight of N = 2 I rows
 * (gate rows 0..I-1, up rows I..N-1), and
 *   y[t][j] = fp16(fp16(silu(g)) * u),  g = (x . W^T + bias)[t][j],  u = (...)[t][I + j]
 * with g and u exactly the fp16 values edgerag_quant_linear would write for the same arguments.
 * y: [M, I] fp16, row stride y_stride. Covered: fp16 x, bits 8 with group_size == K, 16-byte
 * aligned x rows and W, K a multiple of 64 (at least 256), N even, and either 1 <= M <= 64 with
 * N at least 8192 (the streaming GEMV's epilogue), or M > 64 where edgerag_quant_linear's tiled
 * GEMM takes 128-row weight tiles (its epilogue; at most 16 rows past whole 64-row tiles go to
 * the streaming form). Anything else returns EDGERAG_EUNSUPPORTED
 * (edgerag_quant_linear_swiglu_supported says so beforehand); the caller then runs
 * edgerag_quant_linear and edgerag_silu_mul.
 *
 * Replaces `down_proj(F.silu(gate_proj(x)) * up_proj(x))`'s first half (edgerag/core/layers.py:341)
 * for decode batches: the [M, N] projection never goes through HBM, and one launch goes away.
 */
int edgerag_quant_linear_swiglu(const void* x, int32_t x_dtype, int64_t x_stride, int32_t m,
                                int32_t k, const uint8_t* packed, const void* scales_f16,
                                const void* bias_f16, int32_t n, int32_t bits, int32_t group_size,
                                void* y, int64_t y_stride, const float* norm_partials,
                                int32_t norm_parts, float eps, void* stream);
/* 1 when edgerag_quant_linear_swiglu covers (x_dtype, M, K, N, bits, group_size) for 16-byte
 * aligned x rows and W (normed != 0: with a normed input), else 0. */
int edgerag_quant_linear_swiglu_supported(int32_t x_dtype, int32_t m, int32_t k, int32_t n,
                                          int32_t bits, int32_t group_size, int32_t normed);

/*
 * The fused q/k/v quant linear followed by RoPE and the KV append, in one launch. W is the packed
 * INT8 per-channel [n_q_heads | n_kv_heads | n_kv_heads] x head_dim projection (N = heads x
 * head_dim rows). Each projection value is exactly what edgerag_quant_linear writes for the same
 * arguments; the rest is edgerag_rope_append on those values, except that the tables come as one
 * row per token: cos_tok / sin_tok are [M, head_dim] (row t = the table row at token t's
 * position; the caller gathers them, and a NaN row gives that token NaN q and k), fp16. q heads go to q_out (row stride q_stride_tok, head stride
 * head_dim), rotated k and raw v heads to the pools at slots[t] (skipped when negative or
 * outside the pool). Covered: fp16 x, bits 8 with group_size == K, and either 1 <= M <= 64 with
 * K a multiple of 64 (at least 256) handled by at most 8 waves, head_dim a multiple of 32 and N
 * at least 4096 when M <= 16 (the streaming GEMV's epilogue), or M > 64 with head_dim 64 where
 * edgerag_quant_linear's tiled GEMM takes 128-row weight tiles (its epilogue; at most 16 rows
 * past whole 64-row tiles go to the streaming form; cos_tok and sin_tok 8-byte aligned, else
 * EDGERAG_EINVAL). edgerag_quant_linear_rope_append_supported says so beforehand. Anything else
 * returns EDGERAG_EUNSUPPORTED (then run edgerag_quant_linear and edgerag_rope_append).
 *
 * Replaces the decode iteration's q/k/v projections + apply_rope + cache.update's write
 * (edgerag/core/layers.py:93-114, :289-306; edgerag/cache/paged.py:186-206).
 */
int edgerag_quant_linear_rope_append(const void* x, int32_t x_dtype, int64_t x_stride, int32_t m,
                                     int32_t k, const uint8_t* packed, const void* scales_f16,
                                     const void* bias_f16, int32_t bits, int32_t group_size,
                                     const void* cos_tok, const void* sin_tok, int32_t n_q_heads,
                                     int32_t n_kv_heads, int32_t head_dim, void* q_out,
                                     int64_t q_stride_tok, const int32_t* slots, void* key_pool,
                                     void* value_pool, int32_t num_blocks, int32_t block_size,
                                     const float* norm_partials, int32_t norm_parts, float eps,
                                     void* stream);
/* 1 when edgerag_quant_linear_rope_append covers the shape for 16-byte aligned x rows and W
 * (normed != 0: with a normed input). */
int edgerag_quant_linear_rope_append_supported(int32_t x_dtype, int32_t m, int32_t k, int32_t bits,
                                               int32_t group_size, int32_t n_q_heads,
                                               int32_t n_kv_heads, int32_t head_dim,
                                               int32_t normed);

/*
 * Residual add + RMSNorm without launches of their own, for decode batches (M <= 16 tokens, fp16,
 * INT8 per-channel W, the streaming shapes).
 *
 * edgerag_quant_linear_residual is the producer: it computes y = x . W^T (+ bias) exactly as
 * edgerag_quant_linear would, but instead of writing y it adds it to the residual stream in place,
 * hidden[t][j] = fp16(hidden[t][j] + y[t][j]), writes partials[t * P + p] = the fp32 sum of the
 * new hidden values squared over the columns workgroup p owns, and, when next_norm_weight and xw
 * are given, xw[t][j] = fp16(next_norm_weight[j] * hidden[t][j]) (row stride xw_stride). P (the
 * workgroups, at most ceil(N / 8)) goes to *n_parts; partials must hold M * P floats.
 * edgerag_quant_linear_residual_parts returns P for a shape, 0 when it is not covered.
 *
 * The consumer is edgerag_quant_linear_swiglu / edgerag_quant_linear_rope_append with
 * norm_partials != NULL and x = the producer's xw: the projection is then of RMSNorm(hidden) with
 * the weight given to the producer and variance sum_p partials[t][p] / K (summed in a fixed
 * order, so every workgroup and every run gets the same factor). It is computed as
 * r_t * sum_k code * xw[t][k], r_t = rsqrt(variance + eps) applied to the fp32 sum: the reference
 * rounds hidden * r_t to fp16 before the weight multiply, so outputs agree within the linear
 * tolerance, not bit for bit. norm_parts (P) must be at most 256; M at most 16.
 *
 * Replaces `hidden = hidden + out` + RMSNorm.forward between the projections of a decoder layer
 * (edgerag/core/layers.py:40-47, :372-373) for the decode iteration.
 */
int edgerag_quant_linear_residual(const void* x, int32_t x_dtype, int64_t x_stride, int32_t m,
                                  int32_t k, const uint8_t* packed, const void* scales_f16,
                                  const void* bias_f16, int32_t n, int32_t bits,
                                  int32_t group_size, void* hidden, int64_t hidden_stride,
                                  float* partials, int64_t partials_capacity, int32_t* n_parts,
                                  const void* next_norm_weight, void* xw, int64_t xw_stride,
                                  void* stream);
int edgerag_quant_linear_residual_parts(int32_t x_dtype, int32_t m, int32_t k, int32_t n,
                                        int32_t bits, int32_t group_size);

/* ==== Fused elementwise ops of a decoder layer ============================================ */

/*
 * Row-wise residual add + RMSNorm over `rows` rows of `width` elements (`dtype`):
 *   h = x (+ delta)                     rounded to dtype once; written to h_out when delta != NULL
 *   y = weight * dtype(h * rsqrt(mean(h^2) + eps))   variance and scaling in fp32
 * h_out may alias x. Replaces `hidden = hidden + out` followed by RMSNorm.forward
 * (edgerag/core/layers.py:40-47, :372-373). width <= 8192.
 */
int edgerag_rmsnorm(const void* x, int64_t x_stride, const void* delta, int64_t delta_stride,
                    const void* weight, void* h_out, int64_t h_stride, void* y, int64_t y_stride,
                    int32_t rows, int32_t width, float eps, int32_t dtype, void* stream);

/*
 * Embedding lookup + the first layer's RMSNorm, one launch: for t < rows,
 *   h_out[t] = table[ids[t]]            (a copy of the embedding row)
 *   y[t]     = weight * dtype(h * rsqrt(mean(h^2) + eps))   as edgerag_rmsnorm computes it
 * An id outside [0, vocab) has no table row: that row's h and y are written as NaN (the
 * reference's nn.Embedding raises on such an id). Rows must be whole 16-byte chunks, at most
 * 8 x 256 of them (EDGERAG_EUNSUPPORTED otherwise). With positions != NULL the same launch also
 * writes what edgerag_rope_rows writes: cos_out / sin_out [rows, head_dim] = the rows of the
 * [max_pos, head_dim] tables at positions[t] (NaN rows outside the table; head_dim <= 256).
 * Replaces `embed_tokens(input_ids)` (edgerag/core/model.py:109) followed by the first layer's
 * input RMSNorm (edgerag/core/layers.py:27-47), and the step's rotary-row gather.
 */
int edgerag_embed_rmsnorm(const int32_t* ids, int32_t rows, const void* table,
                          int64_t table_stride, int32_t vocab, const void* weight, void* h_out,
                          int64_t h_stride, void* y, int64_t y_stride, int32_t width, float eps,
                          const int32_t* positions, const void* cos_table, const void* sin_table,
                          int32_t max_pos, int32_t head_dim, void* cos_out, void* sin_out,
                          int32_t dtype, void* stream);

/*
 * RoPE on the fused q/k/v projection output and the KV append, in one launch. Row t of qkv holds
 * [n_q_heads | n_kv_heads | n_kv_heads] heads of head_dim elements. For position p =
 * positions[t] in [0, max_pos), q and k heads become dtype(dtype(x * cos[p]) +
 * dtype(rotate_half(x) * sin[p])) with rotate_half(x) = [-x2, x1] (the halves convention); q is
 * written to q_out[t, h, :] (row stride q_stride_tok, head stride head_dim), k and the raw v to
 * key_pool / value_pool [n_kv_heads, num_blocks, block_size, head_dim] at slot slots[t] (skipped
 * when negative or outside the pool). cos/sin tables are [max_pos, head_dim] in dtype. A
 * position outside [0, max_pos) has no table row: that token's q and k are written as NaN (v is
 * still appended), never another position's rotation. The reference computes cos/sin for any
 * position (edgerag/core/layers.py:64-90), so a caller sizes the table for every position it
 * feeds; the positions are on the device, so the check cannot fail the launch itself.
 * Replaces apply_rope + cache.update's write (edgerag/core/layers.py:93-114, :301-306;
 * edgerag/cache/paged.py:186-206).
 */
int edgerag_rope_append(const void* qkv, int64_t qkv_stride, const int32_t* positions,
                        const void* cos_table, const void* sin_table, int32_t max_pos,
                        int32_t n_tokens, int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                        void* q_out, int64_t q_stride_tok, const int32_t* slots, void* key_pool,
                        void* value_pool, int32_t num_blocks, int32_t block_size, int32_t dtype,
                        void* stream);

/*
 * The per-token RoPE rows edgerag_quant_linear_rope_append reads: cos_out[t, :] =
 * cos_table[positions[t], :] and likewise sin, for the n_tokens positions (device int32); a
 * position outside [0, max_pos) gets a row of NaN (that token's q and k then come out NaN). One
 * launch; tables [max_pos, head_dim] and outputs [n_tokens, head_dim] contiguous, in dtype.
 * Replaces the per-call cos/sin of apply_rope (edgerag/core/layers.py:64-90) for one forward.
 */
int edgerag_rope_rows(const int32_t* positions, int32_t n_tokens, const void* cos_table,
                      const void* sin_table, int32_t max_pos, int32_t head_dim, int32_t dtype,
                      void* cos_out, void* sin_out, void* stream);

/*
 * SwiGLU activation of the fused [gate | up] projection: out[t, c] = dtype(dtype(silu(g)) * u),
 * g = gate_up[t, c], u = gate_up[t, intermediate + c]. Replaces silu(gate_proj(x)) * up_proj(x)
 * (edgerag/core/layers.py:341).
 */
int edgerag_silu_mul(const void* gate_up, int64_t gate_up_stride, int32_t n_tokens,
                     int32_t intermediate, void* out, int64_t out_stride, int32_t dtype,
                     void* stream);

/*
 * Greedy token choice over each row of logits [rows, cols] (row stride row_stride elements):
 * out[r] = the first index of the row's maximum, a NaN counting as the maximum (torch.argmax's
 * choice). One workgroup per row. Replaces `int(logits[0, -1].argmax())` of the executor's
 * greedy step (edgerag/serve/executor.py:136, :154) for all emitting requests at once.
 */
int edgerag_argmax_rows(const void* x, int32_t dtype, int32_t rows, int32_t cols,
                        int64_t row_stride, int32_t* out, void* stream);

/*
 * The output head of a decode step and its greedy choice in two launches: for the 1 <= m <= 16
 * emitting rows x [m, k] (fp16, row stride x_stride elements, rows 16-byte aligned) and the fp16
 * lm_head weight [vocab, k] (contiguous, 16-byte aligned; k a multiple of 32):
 *   logits[t][j] = fp16(sum_k x[t][k] * weight[j][k])   (fp32 accumulation; skipped if logits
 *                                                         is NULL; row stride logits_stride)
 *   tokens[t]    = the first j of the maximum of logits[t][:] (a NaN counts as the maximum), the
 *                  choice torch.argmax makes on the fp16 logits.
 * The weight streams from HBM once. workspace (8-byte aligned, any contents) holds one candidate
 * per (row, 64-row slice of the vocabulary): edgerag_lm_head_workspace_bytes(m, vocab) bytes;
 * launches sharing it must be ordered. m > 16 returns EDGERAG_EUNSUPPORTED.
 *
 * Replaces `F.linear(hidden, lm_head)` on the last position (edgerag/core/model.py:150-152) and
 * the greedy `int(logits[0, -1].argmax())` of ModelExecutor.execute
 * (edgerag/serve/executor.py:136, :154) for every emitting request of a step.
 */
int edgerag_lm_head_argmax(const void* x, int64_t x_stride, int32_t m, int32_t k,
                           const void* weight, int32_t vocab, void* logits,
                           int64_t logits_stride, int32_t* tokens, void* workspace,
                           int64_t workspace_bytes, void* stream);
int64_t edgerag_lm_head_workspace_bytes(int32_t m, int32_t vocab);
/* 1 when edgerag_lm_head_argmax takes m rows of width k (1 <= m <= 16, k a multiple of 32 and
 * the m rows staged in 128 KiB of LDS: m * (k / 8 + 1) * 16 bytes), else 0; with 16-byte aligned
 * rows and weight it then accepts the call. */
int edgerag_lm_head_argmax_supported(int32_t m, int32_t k);

#ifdef __cplusplus
}
#endif

#endif /* EDGERAG_AMD_H */
