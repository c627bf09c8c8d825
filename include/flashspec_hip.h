/*
 * flashspec_hip.h — C ABI of libflashspec_hip.so, the MI355X (gfx950) INT8
 * decode-attention library.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t passed
 * as `void*` (NULL = the null stream).  The library never allocates device
 * memory: the caller owns every buffer, including the split-K workspace.
 * Work is enqueued asynchronously on `stream`.
 *
 * Return value: FS_OK (0) on success.  FS_ERR_INVALID means a shape/layout
 * argument was rejected before launch (the reference raises ValueError);
 * FS_ERR_RUNTIME means a HIP runtime failure (the reference raises
 * RuntimeError).  fs_last_error() returns the calling thread's last message.
 *
 * dtype codes: FS_F32 = 0, FS_F16 = 1, FS_BF16 = 2.
 */
#ifndef FLASHSPEC_HIP_H_
#define FLASHSPEC_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FS_OK 0
#define FS_ERR_INVALID 1
#define FS_ERR_RUNTIME 2

#define FS_F32 0
#define FS_F16 1
#define FS_BF16 2

/* Message of the last failed call on this thread ("" if none). */
const char* fs_last_error(void);

/* ABI revision of this header; bumped on any signature change. */
int fs_abi_version(void);

/*
 * Bytes of split-K workspace fs_fused_decode_i8 / fs_paged_decode_i8 need for
 * `rows` (= batch*heads) rows, `max_splits` splits per row and `head_dim`:
 * rows*max_splits*(2 + head_dim) floats.
 */
int64_t fs_decode_workspace_bytes(int64_t rows, int64_t max_splits, int64_t head_dim);

/*
 * Which decode kernel serves a shape: 1 = tiled path, 0 = generic path.  The tiled
 * path takes head_dim a multiple of 16 up to 256 with quant blocks of a multiple of
 * 8 tokens (pages a multiple of the quant block), or one scale per token (quant
 * block 1) on contiguous rows or pages of a multiple of 16 tokens; and head_dim a
 * multiple of 4 from 20 to 252 with quant blocks of a multiple of 16 tokens or one
 * scale per token.  The split plan differs:
 * on the tiled path one split is one workgroup of `waves_per_block` cooperating
 * waves (split_tiles <= 64 * waves_per_block); on the generic path one split is
 * one wave and `waves_per_block` only groups independent waves.
 */
int fs_decode_tiled_path(int head_dim, int page_size, int quant_block);

/*
 * Contiguous INT8 decode attention (one query token per row), split-K with an
 * fp32 log-sum-exp merge.
 *
 * Replaces the launches of _fused_dequant_attention_kernel and
 * _fused_dequant_attention_split_kernel in reference
 * src/flashspec/triton_fused.py:697-734 (launcher
 * _run_fused_dequant_attention_triton, triton_fused.py:604-761).
 *
 *   q        [batch, heads, head_dim]            q_dtype
 *   k/v      values [batch, heads, n_blocks, block_size, head_dim] int8 (uint8 - 128)
 *            scale  [batch, heads, n_blocks] fp32, zero [batch, heads, n_blocks] int16
 *   lengths  [batch] int64 or NULL (NULL = every row uses seq_len)
 *   out      [batch, heads, head_dim]            q_dtype
 *   split_tiles  16-token tiles per split; max_splits >= ceil(ceil(seq_len/16)/split_tiles)
 *   workspace    >= fs_decode_workspace_bytes(batch*heads, max_splits, head_dim) when
 *                max_splits > 1 (else may be NULL).  Rows needing one split are written
 *                to `out` directly; rows needing more leave partial states that
 *                fs_combine_splits merges into `out`.
 *   waves_per_block  1, 2, 4, 8 or 16
 * Results are bit-reproducible: every wave sums its tiles in a fixed order.
 */
int fs_fused_decode_i8(const void* q, int q_dtype,
                       const int8_t* k_values, const float* k_scale, const int16_t* k_zero,
                       const int8_t* v_values, const float* v_scale, const int16_t* v_zero,
                       const int64_t* lengths, void* out,
                       void* workspace, int64_t workspace_bytes,
                       int batch, int heads, int head_dim, int seq_len,
                       int n_blocks, int block_size, float sm_scale,
                       int split_tiles, int max_splits, int waves_per_block, void* stream);

/*
 * Paged INT8 decode attention over a block_table, split-K, fp32 LSE merge.
 *
 * Replaces the launch of _paged_quant_attention_kernel in reference
 * src/flashspec/triton_paged.py:428-434 (launcher
 * _run_paged_quant_attention_triton, triton_paged.py:338-450).
 *
 *   k/v values [num_pages, heads, page_size/quant_block, quant_block, head_dim] int8
 *       scale/zero [num_pages, heads, page_size/quant_block]
 *   block_table [batch, table_cols], int32 (table_index_bytes = 4) or int64 (8);
 *       entries < 0 or >= num_pages mark unallocated pages, whose tokens are masked.
 *   lengths [batch] int64; a row attends to min(lengths[b], max_seq_len) tokens.
 *   Splits, workspace and fs_combine_splits as for fs_fused_decode_i8.
 */
int fs_paged_decode_i8(const void* q, int q_dtype,
                       const int8_t* k_values, const float* k_scale, const int16_t* k_zero,
                       const int8_t* v_values, const float* v_scale, const int16_t* v_zero,
                       const void* block_table, int table_index_bytes, int64_t table_cols,
                       const int64_t* lengths, void* out,
                       void* workspace, int64_t workspace_bytes,
                       int batch, int heads, int head_dim, int64_t num_pages,
                       int page_size, int quant_block, int max_seq_len, float sm_scale,
                       int split_tiles, int max_splits, int waves_per_block, void* stream);

/*
 * Decode with the split merge inside the decode launch (tiled path only; replaces the split
 * kernel plus _combine_splits_kernel pair, reference triton_fused.py:697-744, and gives
 * triton_paged.py:428-434 split-K).  Arguments as fs_fused_decode_i8 / fs_paged_decode_i8 (or
 * their _fp8 / _i8_channel forms, chosen by kv_format: 0 = affine INT8 per block or token,
 * 1 = FP8 E4M3 with NULL zero arrays, 2 = per-channel affine INT8), with the workspace replaced
 * by a merge area of at least fs_decode_merge_area_bytes(batch*heads, max_splits, head_dim)
 * bytes, 256-byte aligned, all zero before its first use.  When rows split, the last split of
 * each row to finish merges the row and writes it; every call leaves the area all zero again,
 * so one area serves any number of later calls (graph replays included) on one stream.  Calls
 * that overlap in time must use different areas.  With max_splits = 1 the area may be NULL.
 */
int64_t fs_decode_merge_area_bytes(int64_t rows, int64_t max_splits, int64_t head_dim);
int fs_fused_decode_merged(const void* q, int q_dtype, int kv_format,
                           const void* k_values, const float* k_scale, const int16_t* k_zero,
                           const void* v_values, const float* v_scale, const int16_t* v_zero,
                           const int64_t* lengths, void* out, void* merge_area, int64_t merge_area_bytes,
                           int batch, int heads, int head_dim, int seq_len, int n_blocks,
                           int block_size, float sm_scale, int split_tiles, int max_splits,
                           int waves_per_block, void* stream);
int fs_paged_decode_merged(const void* q, int q_dtype, int kv_format,
                           const void* k_values, const float* k_scale, const int16_t* k_zero,
                           const void* v_values, const float* v_scale, const int16_t* v_zero,
                           const void* block_table, int table_index_bytes, int64_t table_cols,
                           const int64_t* lengths, void* out, void* merge_area, int64_t merge_area_bytes,
                           int batch, int heads, int head_dim, int64_t num_pages,
                           int page_size, int quant_block, int max_seq_len, float sm_scale,
                           int split_tiles, int max_splits, int waves_per_block, void* stream);

/*
 * fs_paged_decode_i8 (affine INT8 per block or token, tiled path) with the requests dispatched in
 * a caller-given order: workgroups take request request_order[i] in the place of request i, so a
 * caller that knows the lengths can start the longest rows first and leave short ones for the
 * last round of workgroups (a 64-request ragged serving batch: 600 instead of 611 us).  The
 * outputs do not depend on the order.  request_order is a device int32 permutation of
 * [0, batch), or NULL for the natural order; an entry outside [0, batch) keeps the natural
 * request, and a repeated entry computes that request twice and leaves another unwritten.  Rows
 * that split merge through `merge_area` when it is given (fs_paged_decode_merged's contract),
 * else through `workspace` and a merge launch made here.  No counterpart in the reference
 * (its Triton grid runs one program per (b, h) in index order, triton_paged.py:428-434).
 */
int fs_paged_decode_ordered(const void* q, int q_dtype,
                            const int8_t* k_values, const float* k_scale, const int16_t* k_zero,
                            const int8_t* v_values, const float* v_scale, const int16_t* v_zero,
                            const void* block_table, int table_index_bytes, int64_t table_cols,
                            const int64_t* lengths, const int32_t* request_order, void* out,
                            void* workspace, int64_t workspace_bytes,
                            void* merge_area, int64_t merge_area_bytes,
                            int batch, int heads, int head_dim, int64_t num_pages,
                            int page_size, int quant_block, int max_seq_len, float sm_scale,
                            int split_tiles, int max_splits, int waves_per_block, void* stream);

/*
 * fs_paged_decode_i8 without a workspace argument, for callers that cannot allocate device
 * memory (code under graph capture, serving loops that forbid allocation).  No counterpart in
 * the reference.  When rows split (max_splits > 1) the split-K partials go to a device array
 * inside the library, one per GPU, of fs_noalloc_scratch_bytes() bytes (16 MiB), and this call
 * also launches the split merge (no separate fs_combine_splits).  Plans whose partials,
 * fs_decode_workspace_bytes(batch*heads, max_splits, head_dim), exceed that size are rejected
 * with FS_ERR_INVALID.  Nothing needs clearing between calls: every split writes its partials
 * before the merge reads them.  All calls on one GPU share its array: calls that overlap on one
 * GPU (other streams, other host threads) race.
 */
int fs_paged_decode_i8_noalloc(const void* q, int q_dtype,
                               const int8_t* k_values, const float* k_scale, const int16_t* k_zero,
                               const int8_t* v_values, const float* v_scale, const int16_t* v_zero,
                               const void* block_table, int table_index_bytes, int64_t table_cols,
                               const int64_t* lengths, void* out,
                               int batch, int heads, int head_dim, int64_t num_pages,
                               int page_size, int quant_block, int max_seq_len, float sm_scale,
                               int split_tiles, int max_splits, int waves_per_block, void* stream);

/* Bytes of the device array behind fs_paged_decode_i8_noalloc (per GPU). */
int64_t fs_noalloc_scratch_bytes(void);

/*
 * Speculative-decoding tree verification over a paged INT8 prefix.  Request b has `nodes`
 * draft nodes in topological order; node n attends to the prefix tokens [0, lengths[b]) of
 * the paged cache and to the draft tokens on its path to the root (n, parents[b, n],
 * parents[b, parents[b, n]], ... until -1).  The prefix part leaves split partials per
 * (b, n, h) row in `workspace`; a tail kernel merges them with the path tokens (fp32 online
 * softmax) and writes `out`.  Prefix kernels (`prefix_kernel`):
 *   1 = the paged decode with one query row per node (any store the decode serves);
 *   2 = the multi-query kernel: one wave reads each 16-token tile once for the 16 or 32
 *       nodes of its workgroup with MFMA products (fs_tree_mfma_path() stores;
 *       waves_per_block 1/2/4/8, <= 4 for head_dim 256), the node count being
 *       fs_tree_nodes_per_workgroup() for the current device; split plan over
 *       batch*heads*ceil(nodes/node count) workgroups per split;
 *   3, 4 = 2 with 16- or 32-node workgroups (32 where fs_tree_nodes_per_workgroup() can
 *       return it for some grid; FS_ERR_INVALID otherwise);
 *   0 = 2 where fs_tree_mfma_path() holds, else 1.
 * With the multi-query kernel, one split (max_splits == 1) and drafts in q's dtype, the prefix
 * kernel finishes the rows itself (path tokens and output; no tail launch, workspace unused).
 *   q, out          [batch, nodes, heads, head_dim]  q_dtype
 *   draft_k/draft_v [batch, nodes, heads, head_dim]  draft_dtype (unquantized)
 *   parents         [batch, nodes] int64, parents[b, n] in [-1, n) (the caller validates;
 *                   the kernel ends a path at any entry outside that range)
 *   workspace       >= fs_decode_workspace_bytes(batch*nodes*heads, max_splits, head_dim)
 *   other arguments as for fs_paged_decode_i8 (split plan for batch*nodes*heads rows).
 * No counterpart in the reference, which plans this kernel (doc/TODO.MD:186-237) without
 * implementing it; a chain of nodes reduces to paged decode over prefix + path.
 */
int fs_tree_verify_i8(const void* q, int q_dtype,
                      const int8_t* k_values, const float* k_scale, const int16_t* k_zero,
                      const int8_t* v_values, const float* v_scale, const int16_t* v_zero,
                      const void* block_table, int table_index_bytes, int64_t table_cols,
                      const int64_t* lengths, const void* draft_k, const void* draft_v, int draft_dtype,
                      const int64_t* parents, void* out, void* workspace, int64_t workspace_bytes,
                      int batch, int nodes, int heads, int head_dim, int64_t num_pages,
                      int page_size, int quant_block, int max_seq_len, float sm_scale,
                      int split_tiles, int max_splits, int waves_per_block, int prefix_kernel,
                      void* stream);

/*
 * fs_tree_verify_i8 over an FP8 E4M3 store (fs_quantize_pages_fp8 layout: codes and fp32 scales,
 * no zero points; every prefix kernel, the multi-query one converting the codes exactly to its
 * fp16 operands) and over a per-channel INT8 store (fs_quantize_pages_i8_channel layout: scale /
 * zero [num_pages, heads, page_size/quant_block, head_dim]; the row-kernel prefix only,
 * prefix_kernel 0 or 1, 2-4 being rejected).  Arguments as for fs_tree_verify_i8.  No
 * counterpart in the reference.
 */
int fs_tree_verify_fp8(const void* q, int q_dtype,
                       const uint8_t* k_values, const float* k_scale,
                       const uint8_t* v_values, const float* v_scale,
                       const void* block_table, int table_index_bytes, int64_t table_cols,
                       const int64_t* lengths, const void* draft_k, const void* draft_v, int draft_dtype,
                       const int64_t* parents, void* out, void* workspace, int64_t workspace_bytes,
                       int batch, int nodes, int heads, int head_dim, int64_t num_pages,
                       int page_size, int quant_block, int max_seq_len, float sm_scale,
                       int split_tiles, int max_splits, int waves_per_block, int prefix_kernel,
                       void* stream);
int fs_tree_verify_i8_channel(const void* q, int q_dtype,
                              const int8_t* k_values, const float* k_scale, const int16_t* k_zero,
                              const int8_t* v_values, const float* v_scale, const int16_t* v_zero,
                              const void* block_table, int table_index_bytes, int64_t table_cols,
                              const int64_t* lengths, const void* draft_k, const void* draft_v, int draft_dtype,
                              const int64_t* parents, void* out, void* workspace, int64_t workspace_bytes,
                              int batch, int nodes, int heads, int head_dim, int64_t num_pages,
                              int page_size, int quant_block, int max_seq_len, float sm_scale,
                              int split_tiles, int max_splits, int waves_per_block, int prefix_kernel,
                              void* stream);

/*
 * Tree verification on the multi-query kernel with its split merge inside the launch: rows
 * whose prefix splits (max_splits > 1) publish per-node states to `merge_area`
 * (fs_paged_decode_merged's contract: zero-filled before the first call, left zero by every
 * call, fs_decode_merge_area_bytes(batch * nodes * heads, max_splits, head_dim) bytes, one
 * area per stream), and the last split of each (request, head, node group) merges them and
 * finishes the rows (path tokens, output) -- no workspace and no tail launch.  kv_format 0 =
 * affine INT8 per block or token, 1 = FP8 E4M3 (zero arrays unused); drafts in q's dtype;
 * nodes_per_workgroup 0 (the library's choice), 16 or 32.  The in-launch merge holds at most
 * 272 splits per row at head_dim 64, 528 at 128 and 520 at 256 (two floats per node and split
 * in the workgroup's LDS accumulator); larger max_splits with max_splits > 1 are rejected
 * (FS_ERR_INVALID).  Other arguments as for fs_tree_verify_i8.  No counterpart in the reference
 * (its Kernel 3 is planned only, doc/TODO.MD:186-237).
 */
int fs_tree_verify_merged(const void* q, int q_dtype, int kv_format,
                          const void* k_values, const float* k_scale, const int16_t* k_zero,
                          const void* v_values, const float* v_scale, const int16_t* v_zero,
                          const void* block_table, int table_index_bytes, int64_t table_cols,
                          const int64_t* lengths, const void* draft_k, const void* draft_v,
                          const int64_t* parents, void* out, void* merge_area, int64_t merge_area_bytes,
                          int batch, int nodes, int heads, int head_dim, int64_t num_pages,
                          int page_size, int quant_block, int max_seq_len, float sm_scale,
                          int split_tiles, int max_splits, int waves_per_block,
                          int nodes_per_workgroup, void* stream);

/*
 * 1 when fs_tree_verify_i8 can run its multi-query prefix kernel on this store: head_dim 64,
 * 128 or 256, page_size a multiple of 16, quant_block 1 or a multiple of 16 dividing the
 * page.  No counterpart in the reference (tree verification is not implemented there).
 */
int fs_tree_mfma_path(int head_dim, int page_size, int quant_block);

/*
 * Draft nodes one workgroup of the multi-query tree kernel serves (each of its waves reads a
 * tile once for all of them), as fs_tree_verify_i8 with prefix_kernel 0 or 2 chooses them on a
 * device of `cu_count` CUs: 32 when a wave has the registers for two 16-node groups (head_dim
 * 64, or head_dim 128 with fp16 / bf16 queries and quant_block > 1), nodes > 16, and
 * batch_heads * ceil(nodes / 16) workgroups would exceed cu_count; else 16.  The split plan
 * counts batch_heads * ceil(nodes / this) workgroups per split.  No counterpart in the
 * reference.
 */
int fs_tree_nodes_per_workgroup(int head_dim, int nodes, int q_dtype, int quant_block, int64_t batch_heads,
                                int cu_count);

/*
 * Merge the per-split partial states a decode call with max_splits > 1 left in
 * `workspace`, for the rows that needed more than one split.  Replaces _combine_splits_kernel
 * (reference src/flashspec/triton_fused.py:445-503).  `lengths` may be NULL;
 * with it each row merges ceil(min(len,seq_len)/16/split_tiles) splits (>= 1).
 */
int fs_combine_splits(const void* workspace, const int64_t* lengths, void* out, int out_dtype,
                      int batch, int heads, int head_dim, int seq_len,
                      int split_tiles, int max_splits, void* stream);

/*
 * Affine per-block INT8 quantization, bit-exact with the float32 op sequence
 * of reference src/flashspec/quant.py:94-165 (replaces its eager chain).
 *   x [outer, seq_len, head_dim] x_dtype (contiguous)
 *   values [outer, ceil(seq_len/block), block, head_dim] int8
 *   scale/zero [outer, ceil(seq_len/block)] fp32 / int16
 */
int fs_quantize_i8(const void* x, int x_dtype, int64_t outer, int seq_len, int head_dim,
                   int block_size, int8_t* values, float* scale, int16_t* zero, void* stream);

/*
 * Symmetric absmax INT8 with one fp32 scale per token row (per head):
 *   scale = max(absmax(row) / 127, 1e-8), q = clamp(rint(x / scale), -127, 127)
 * written in the affine layout of fs_quantize_i8 with block size 1 and zero point 128, so
 * every decode entry point reads it (the tiled kernels with one parameter set per token).
 *   x [rows, head_dim] x_dtype; values [rows, head_dim] int8 (= q); scale / zero [rows].
 * No counterpart in the reference, whose quantizer is the affine per-block one: a second
 * KV format offered beside it (symmetric absmax INT8, one fp32 scale per token per head).
 */
int fs_quantize_sym_i8(const void* x, int x_dtype, int64_t rows, int head_dim,
                       int8_t* values, float* scale, int16_t* zero, void* stream);

/*
 * FP8 E4M3 (OCP "e4m3fn") KV format: per block of block_size tokens x head_dim (zero-padded
 * like fs_quantize_i8), one fp32 scale and no zero point:
 *   scale = max(absmax / 448, 1e-8), code = E4M3 round-to-nearest-even of clamp(x / scale, ±448)
 * values [outer, nb, block_size, head_dim] codes (torch.float8_e4m3fn bytes), scale
 * [outer, nb]; `zero` (may be null) is filled with 0 so the INT8 layout is kept.
 * fs_quantize_pages_fp8 is fs_quantize_pages_i8's page-store form (block = page).
 * No counterpart in the reference, which lists FP8 among the KV formats to compare
 * (doc/TODO.MD:241-255) without implementing it.
 */
int fs_quantize_fp8(const void* x, int x_dtype, int64_t outer, int seq_len, int head_dim,
                    int block_size, uint8_t* values, float* scale, int16_t* zero, void* stream);
int fs_quantize_pages_fp8(const void* x, int x_dtype, int batch, int heads, int seq_len,
                          int head_dim, int page_size, const int64_t* page_src, int64_t num_pages,
                          uint8_t* values, float* scale, int16_t* zero, void* stream);
/* float32(code) * scale, padding cropped; out [outer, seq_len, head_dim] out_dtype. */
int fs_dequantize_fp8(const uint8_t* values, const float* scale, int64_t outer, int n_blocks,
                      int block_size, int head_dim, int seq_len, void* out, int out_dtype,
                      void* stream);

/*
 * Decode attention over FP8 E4M3 stores: fs_fused_decode_i8 / fs_paged_decode_i8 with FP8
 * codes and per-block (or per-token, block 1) scales and no zero points; same kernels, plan,
 * workspace and fs_combine_splits.  No counterpart in the reference (see fs_quantize_fp8).
 */
int fs_fused_decode_fp8(const void* q, int q_dtype, const uint8_t* k_values, const float* k_scale,
                        const uint8_t* v_values, const float* v_scale, const int64_t* lengths,
                        void* out, void* workspace, int64_t workspace_bytes, int batch, int heads,
                        int head_dim, int seq_len, int n_blocks, int block_size, float sm_scale,
                        int split_tiles, int max_splits, int waves_per_block, void* stream);
int fs_paged_decode_fp8(const void* q, int q_dtype, const uint8_t* k_values, const float* k_scale,
                        const uint8_t* v_values, const float* v_scale, const void* block_table,
                        int table_index_bytes, int64_t table_cols, const int64_t* lengths,
                        void* out, void* workspace, int64_t workspace_bytes, int batch, int heads,
                        int head_dim, int64_t num_pages, int page_size, int quant_block,
                        int max_seq_len, float sm_scale, int split_tiles, int max_splits,
                        int waves_per_block, void* stream);

/*
 * Per-channel affine INT8 KV format: per block of block_size tokens, one scale / zero point per
 * channel, each channel column quantized with fs_quantize_i8's float32 op sequence; scale / zero
 * [outer, nb, head_dim] (pages: [num_pages, heads, head_dim]).  The decode entry points take the
 * arguments of fs_fused_decode_i8 / fs_paged_decode_i8 with those arrays; their tiled path needs
 * quant blocks of a multiple of 16 tokens (fs_decode_tiled_path_channel), workgroups of at most 8
 * waves, and otherwise runs the element-wise kernel.  No counterpart in the reference, which lists
 * per-channel scales among the KV formats to compare (doc/TODO.MD:241-255).
 */
int fs_quantize_i8_channel(const void* x, int x_dtype, int64_t outer, int seq_len, int head_dim,
                           int block_size, int8_t* values, float* scale, int16_t* zero, void* stream);
int fs_quantize_pages_i8_channel(const void* x, int x_dtype, int batch, int heads, int seq_len,
                                 int head_dim, int page_size, const int64_t* page_src,
                                 int64_t num_pages, int8_t* values, float* scale, int16_t* zero,
                                 void* stream);
int fs_fused_decode_i8_channel(const void* q, int q_dtype,
                               const int8_t* k_values, const float* k_scale, const int16_t* k_zero,
                               const int8_t* v_values, const float* v_scale, const int16_t* v_zero,
                               const int64_t* lengths, void* out, void* workspace,
                               int64_t workspace_bytes, int batch, int heads, int head_dim,
                               int seq_len, int n_blocks, int block_size, float sm_scale,
                               int split_tiles, int max_splits, int waves_per_block, void* stream);
int fs_paged_decode_i8_channel(const void* q, int q_dtype,
                               const int8_t* k_values, const float* k_scale, const int16_t* k_zero,
                               const int8_t* v_values, const float* v_scale, const int16_t* v_zero,
                               const void* block_table, int table_index_bytes, int64_t table_cols,
                               const int64_t* lengths, void* out, void* workspace,
                               int64_t workspace_bytes, int batch, int heads, int head_dim,
                               int64_t num_pages, int page_size, int quant_block, int max_seq_len,
                               float sm_scale, int split_tiles, int max_splits, int waves_per_block,
                               void* stream);
int fs_decode_tiled_path_channel(int head_dim, int page_size, int quant_block);

/*
 * Dequantize ((v + 128) - zero) * scale and crop the padding.  Replaces
 * reference src/flashspec/quant.py:168-204.
 *   out [outer, seq_len, head_dim] out_dtype
 */
int fs_dequantize_i8(const int8_t* values, const float* scale, const int16_t* zero,
                     int64_t outer, int n_blocks, int block_size, int head_dim, int seq_len,
                     void* out, int out_dtype, void* stream);

/*
 * Quantize dense K or V [batch, heads, seq_len, head_dim] straight into the
 * physical page store [num_pages = batch*ceil(seq_len/page), heads, page, head_dim]
 * (one quant block per page), gathering page j from batch-major logical page
 * page_src[j] (NULL = identity).  Replaces the permute/pad/index/quantize chain
 * of PagedKVCache.from_dense, reference src/flashspec/paged.py:343-412.
 */
int fs_quantize_pages_i8(const void* x, int x_dtype, int batch, int heads, int seq_len,
                         int head_dim, int page_size, const int64_t* page_src, int64_t num_pages,
                         int8_t* values, float* scale, int16_t* zero, void* stream);

/*
 * Rewrite whole pages: for each listed page, start from zeros (fresh[i] != 0)
 * or from the dequantized old page (all rows, stale ones included), overwrite
 * the rows that row_src names with new tokens, requantize the page per head
 * (quant block = page_size) and store it.
 *
 * Replaces PagedKVCache.append's dequantize/write/requantize
 * (reference src/flashspec/paged.py:498-550) and the allocator's per-page
 * path (paged.py:92-136, 226-255).
 *
 *   in_*     old store [in_pages, heads, page/in_quant_block, in_quant_block, head_dim]
 *   out_*    new store [*, heads, 1, page, head_dim]; may alias in_* (in place)
 *   pages    [n_pages] int64 page ids to rewrite, or NULL = pages 0..n_pages-1
 *   fresh    [n_pages] uint8 or NULL (= none fresh); pages >= in_pages are fresh
 *   row_src  [n_pages, page] int32: -1 keeps the row, else n*src_tokens + t
 *            selects token t of entry n of src [*, heads, src_tokens, head_dim]
 */
int fs_update_pages_i8(const int8_t* in_values, const float* in_scale, const int16_t* in_zero,
                       int64_t in_pages, int in_quant_block,
                       int8_t* out_values, float* out_scale, int16_t* out_zero,
                       const int64_t* pages, const uint8_t* fresh, int64_t n_pages,
                       const int32_t* row_src, const void* src, int src_dtype, int src_tokens,
                       int heads, int page_size, int head_dim, void* stream);

/* One decode step's append, device-resident: for every request b, the token
 * k_new/v_new[b] ([batch, heads, 1, head_dim], dtype src_dtype) goes to position
 * pos = lengths_in[b], i.e. row pos % page_size of physical page block_table[b, pos / page_size];
 * that page's [heads] groups are dequantized (stale rows included), the row is replaced and
 * the page is requantized in place (quant block == page_size), for K and V in one launch.
 * lengths_out[b] = pos + 1, or pos when the table entry is -1 / out of range (the token is
 * then dropped and nothing is written).  `dropped` (NULL, or one unsigned of device memory the
 * caller zeroes) counts the dropped tokens, one per request, with device atomics: the reference
 * allocator raises instead of dropping (paged.py:89-90, 222-224), so a caller that must not lose
 * tokens checks it.  lengths_in and lengths_out must differ; the caller
 * fills the table entry of a page before the step that first writes it.
 * Replaces PagedKVAllocator.append_batch for one token per request
 * (reference src/flashspec/paged.py:108-144, with page reads at :226-245 and writes at :247-255). */
int fs_append_tokens_i8(const void* k_new, const void* v_new, int src_dtype,
                        int8_t* k_values, float* k_scale, int16_t* k_zero,
                        int8_t* v_values, float* v_scale, int16_t* v_zero, int64_t num_pages,
                        const void* block_table, int table_index_bytes, int table_cols,
                        const int64_t* lengths_in, int64_t* lengths_out,
                        int batch, int heads, int head_dim, int page_size, unsigned* dropped,
                        void* stream);

/* One serving decode step in one launch: fs_append_tokens_i8 followed by paged decode attention
 * over the advanced lengths, with the append done inside the decode kernel.  For every request b,
 * the wave whose tile holds position pos = lengths_in[b] requantizes that page (the op sequence
 * and results of fs_append_tokens_i8, bit for bit) and attends over it from registers; every row
 * covers pos + 1 tokens.  lengths_out[b] = pos + 1, or pos when the page is not backed (table
 * entry -1 or out of range) or pos >= max_seq_len -- such a token is dropped, stays masked and
 * counts into `dropped` (NULL or a caller-zeroed device unsigned, as for fs_append_tokens_i8).
 * Needs 16-token pages holding one quant block, head_dim 64 / 128 / 256, and k_new / v_new
 * ([batch, heads, 1, head_dim]) in q's dtype; max_seq_len must exceed every lengths_in[b] for
 * the token to be kept.  Rows that split merge through `merge_area` when it is given
 * (fs_paged_decode_merged's contract), else through `workspace` and a merge launch made here.
 * The op order is append-then-attend (standard decode: the new token's K/V are known before
 * its attention), the order of DecodeBatch.step; the reference's serving loop attends first and
 * appends K/V made from the attention output (serving.py:126-163), which a caller gets from the
 * paged decode followed by fs_append_tokens_i8.  Replaces the PagedKVAllocator.append_batch +
 * paged attention pair of a decode step (reference src/flashspec/paged.py:108-144). */
int fs_paged_decode_append_i8(const void* q, int q_dtype, const void* k_new, const void* v_new,
                              int8_t* k_values, float* k_scale, int16_t* k_zero,
                              int8_t* v_values, float* v_scale, int16_t* v_zero,
                              const void* block_table, int table_index_bytes, int64_t table_cols,
                              const int64_t* lengths_in, int64_t* lengths_out, void* out,
                              void* workspace, int64_t workspace_bytes,
                              void* merge_area, int64_t merge_area_bytes,
                              int batch, int heads, int head_dim, int64_t num_pages, int page_size,
                              int max_seq_len, float sm_scale, int split_tiles, int max_splits,
                              int waves_per_block, unsigned* dropped, void* stream);

/* Measurement helper with no counterpart in the reference: one plain streaming read of
 * `bytes` (a positive multiple of 16, `src` 16-byte aligned) by `blocks` workgroups of 256
 * lanes, non-temporal 16-byte loads in a grid-stride loop (the decode kernels' load form).  Its rate is the practical HBM read ceiling that
 * bench.py sets beside the decode kernel's; `sink` (4 bytes of device memory) is written only
 * if the XOR of everything read matches a fixed word. */
int fs_stream_read(const void* src, int64_t bytes, unsigned* sink, int blocks, void* stream);

/*
 * Measurement helper (no reference counterpart): streams src_bytes from src with 16-byte
 * non-temporal loads and writes src_bytes / 2 to dst (two bytes of every four), in `blocks`
 * workgroups of 256 lanes: the traffic of an fp16 -> int8 pass with no arithmetic, whose rate is
 * the practical ceiling of the quantizers.
 */
int fs_stream_copy_half(const void* src, int64_t src_bytes, void* dst, int blocks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLASHSPEC_HIP_H_ */
