// Paged / contiguous INT8 K/V store addressing and the decode launch parameters shared by the
// decode kernels (fs_decode.hip) and the multi-query tree-verification kernel (fs_tree.hip).
#pragma once

#include "fs_common.h"

namespace fs {

constexpr int kMaxWaves = 16;       // waves per workgroup on the tiled path
constexpr int kMaxTilesPerWave = 64;  // per split and wave: one metadata lane per tile
constexpr float kRescaleSlack = 8.0f;  // running max may lag the true max by 2^8
constexpr int kXcds = 8;  // MI355X: accelerator complex dies, each with its own L2

// How a tile finds its quantization parameters (scale / zero point).
enum QuantMode : int {
  kQmBlock = 0,  // quant block a multiple of 16 tokens: one entry per tile
  kQmSub = 1,    // quant block an odd multiple of 8 tokens (or 8-token pages): one per 8-token half
  kQmToken = 2,  // one entry per token (quant block 1, e.g. symmetric per-token INT8)
  kQmChannel = 3,  // per quant block (a multiple of 16 tokens) one entry per channel
  kQmChannelBlocks = 4,  // kQmChannel with quant blocks of >= 2 tiles: waves take whole blocks
  // kQmBlock / kQmToken for a head_dim that is a multiple of 4 but not of 16 (>= 20): the lane
  // whose 16 dims straddle the row end loads the row's last 16 bytes and uses their upper part
  kQmBlockTail = 5,
  kQmTokenTail = 6,
  // kQmBlock (paged, 16-token pages holding one quant block, head_dim 64 / 128 / 256) with one
  // decode token appended to every request inside the launch (fs_paged_decode_append_i8)
  kQmBlockAppend = 7,
};

// Value format of the K/V store: affine INT8 (values int8 = u - 128, scale, zero point) or FP8
// E4M3 codes with a scale and no zero point (the zero arrays are all 0 and unused).
enum ValueFormat : int {
  kVfInt8 = 0,
  kVfFp8 = 1,
};

struct DecodeParams {
  const void* q;
  const int8_t* kv[2];
  const float* sc[2];
  const int16_t* zp[2];
  const void* table;
  int64_t table_cols;
  int table_bytes;
  const int64_t* lengths;
  void* out;
  float* part_ml;   // [rows, max_splits, 2] (max in log2 units, denominator)
  float* part_acc;  // [rows, max_splits, D]
  int rows, heads, head_dim;
  int seq_len;
  int64_t num_pages;
  int n_blocks;
  int quant_block;
  int page_size;
  int split_tiles, max_splits;
  float qk_scale;  // sm_scale * log2(e)
  // Tree verification: nq query rows per (request, head), rows ordered (b, n, h); the decode
  // writes split partials for every row (force_partials) for the tree-tail merge.
  int nq;
  int force_partials;
  int vfmt;  // ValueFormat
  int per_channel;  // scale / zero hold head_dim entries per quant block (INT8 only)
  // Multi-query tree kernel with one split: it finishes the rows itself (path tokens from
  // draft_k / draft_v, which then have q's dtype, and parents) instead of leaving partials.
  int fuse_tail;
  int pace_waves;  // multi-query tree kernel: the waves sharing a SIMD pace each other
  const void* draft_k;
  const void* draft_v;
  const int64_t* parents;
  // In-kernel split merge (tiled kernel, merge_count != nullptr): a zero-filled area of per-row
  // arrival counts [rows] and tagged partial states [rows, max_splits, D + 2] (64-bit words, tag 1 in
  // the upper half); the last split of a row to arrive merges the row and zeroes what it used.
  unsigned* merge_count;
  unsigned long long* merge_slots;
  // The launch's tag in the upper half of its merge words (never 0, taken from a per-process counter
  // at every launch): a word that a split of an earlier launch stored after that launch had given up
  // waiting for it and cleared the area carries another tag, so it never passes for a later launch's.
  unsigned merge_tag;
  // One-token append fused into the paged decode (kQmBlockAppend): `lengths` holds each request's
  // position before the append; the new K / V rows append_k / append_v [rows, head_dim] (q's
  // dtype) go into the page at that position, which is requantized in place, and the advanced
  // lengths go to lengths_out.
  const void* append_k;
  const void* append_v;
  int64_t* lengths_out;
  unsigned* dropped;  // counts the appended tokens that were not stored (NULL: not counted)
  // Dispatch order of the requests (tiled decode): workgroups take request request_order[i] in the
  // place of request i (a permutation of [0, batch); NULL = natural order).  Serving batches pass
  // their requests longest first, so the last round of workgroups holds short rows.
  const int32_t* request_order;
};

// Words of the in-kernel split merge (decode rows and tree verification): a split's state goes out
// as 64-bit words with the launch's tag in the upper half (DecodeParams::merge_tag), stored with
// relaxed agent-scope atomic stores, so a reader sees a word whole or not at all and waits on the
// tag, not on a fence; the waits are bounded by kMergeSpins (a row whose words never land is written
// as NaN).
constexpr int kMergeSpins = 1 << 14;

__device__ __forceinline__ void publish(unsigned long long* w, float x, unsigned tag) {
  __hip_atomic_store(w, ((unsigned long long)tag << 32) | __float_as_uint(x), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void clear_word(unsigned long long* w) {
  __hip_atomic_store(w, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned long long load_word(const unsigned long long* w) {
  return __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The value of word w, given a first load v of it: reloads until it carries the launch's tag.
__device__ __forceinline__ float settle_word(unsigned long long v, const unsigned long long* w, bool& ok,
                                            unsigned tag) {
  for (int n = 0; (unsigned)(v >> 32) != tag && n < kMergeSpins; ++n) {
    __builtin_amdgcn_s_sleep(1);
    v = load_word(w);
  }
  ok = ok && (unsigned)(v >> 32) == tag;
  return __uint_as_float((unsigned)v);
}

// Bytes of a merge area: the counts padded to 256 bytes, then the slots.
__host__ __device__ inline int64_t merge_area_bytes(int64_t rows, int64_t max_splits, int64_t head_dim) {
  return (rows * 4 + 255) / 256 * 256 + rows * max_splits * (head_dim + 2) * 8;
}

__device__ __forceinline__ int queries_per_head(const DecodeParams& p) { return p.nq > 1 ? p.nq : 1; }

// The dispatcher hands workgroups to the XCDs round-robin (workgroup i to XCD i % 8), each with its
// own L2.  xcd_chunked_unit renumbers a 1-D grid of `units` so that XCD x takes the x-th eighth of
// the units in order (the tree kernel orders its units so that an eighth is a slab of heads).
__device__ __forceinline__ int xcd_chunked_unit(int bid, int units) {
  const int per = units / kXcds, rem = units - per * kXcds;
  const int x = bid % kXcds, k = bid / kXcds;
  return x * per + min(x, rem) + k;
}

__device__ __forceinline__ int row_length(const int64_t* lengths, int b, int seq_len) {
  if (lengths == nullptr) return seq_len;
  const int64_t l = lengths[b];
  return (int)(l < 0 ? 0 : (l < (int64_t)seq_len ? l : (int64_t)seq_len));
}

// Row length once the fused append (kQmBlockAppend) has added the token at position lengths[b].
__device__ __forceinline__ int row_length_after_append(const int64_t* lengths, int b, int seq_len) {
  const int64_t pos = lengths[b];
  const int64_t l = pos >= 0 ? pos + 1 : 0;
  return (int)(l < (int64_t)seq_len ? l : (int64_t)seq_len);
}

__device__ __forceinline__ int row_splits(int len, int split_tiles) {
  const int tiles = (len + kTile - 1) / kTile;
  const int n = (tiles + split_tiles - 1) / split_tiles;
  return n < 1 ? 1 : n;
}

// Rotation of a wave's tile order for a row of request b (nk tiles): the wave takes its first tile
// (the one contiguous rows load before the row length is known), then its others from position
// 1 + ((b + 8 * split) mod (nk - 1)) on, wrapping around.  All requests walking their tiles in step would have
// the whole GPU read, at any moment, one page of each request; in the contiguous page layout those
// pages sit a fixed power-of-two stride apart (one request's pages apart), and on some physical
// placements such a set falls on few HBM channels: measured on one MI355X, 2 of 8 identical
// metric-shape caches then read 43.4 us against 40.5-40.8 us for the others, reproducibly, while
// shuffled pages (41.9 us) and contiguous rows (40.0-40.7 us) did not vary; with the rotation all
// eight read 40.9-41.7 us.  The splits of one row sit a power-of-two stride apart as well (one split's
// pages) and get rotations of their own.  The rotation depends on the request and the split alone
// and applies to every layout (contiguous rows included), so a row of a given launch plan gives
// bit-identical results in any layout.
__device__ __forceinline__ int tile_rotation(int b, int split, int nk) { return nk > 2 ? (b + 8 * split) % (nk - 1) : 0; }

// The wave's k-th tile in the rotated order (k >= nk: none, k itself).
__device__ __forceinline__ int tile_in_order(int k, int rot, int nk) {
  const int kk = k + rot;
  return k == 0 || k >= nk ? k : (kk >= nk ? kk - (nk - 1) : kk);
}

__device__ __forceinline__ int64_t table_entry(const DecodeParams& p, int b, int64_t col) {
  if (p.table_bytes == 4) return (int64_t)((const int32_t*)p.table)[(int64_t)b * p.table_cols + col];
  return ((const int64_t*)p.table)[(int64_t)b * p.table_cols + col];
}

// Sequence tile `tile` (16 tokens) of (b, h): `data` indexes 16*D-byte tiles of the value
// store, `meta` the scale / zero entries (one per quant block; a quant block is a multiple
// of 16 tokens on this path, so a tile never straddles two).  data = -1 when the tile is
// not backed by an allocated page.
struct TileIndex {
  int data, meta;
};

template <bool PAGED>
__device__ __forceinline__ TileIndex tile_index(const DecodeParams& p, int b, int h, int row, int tile) {
  const int tpq = p.quant_block / kTile;  // tiles per quant block
  if constexpr (PAGED) {
    const int tpp = p.page_size / kTile;
    const int lp = tile / tpp;
    const int sub = tile - lp * tpp;
    if (lp >= p.table_cols) return {-1, 0};
    const int64_t pg = table_entry(p, b, lp);
    if (pg < 0 || pg >= p.num_pages) return {-1, 0};
    const int64_t ph = pg * p.heads + h;
    return {(int)(ph * tpp + sub), (int)(ph * (tpp / tpq) + sub / tpq)};
  } else {
    return {row * p.n_blocks * tpq + tile, row * p.n_blocks + tile / tpq};
  }
}

// The second half of tile_index<true>, for a kernel that loads the table entries itself: the
// tile of head h that table entry pg (-1: none) names for sequence tile `tile`.
__device__ __forceinline__ TileIndex tile_from_page(const DecodeParams& p, int h, int tile, int64_t pg) {
  const int tpq = p.quant_block / kTile, tpp = p.page_size / kTile;
  const int sub = tile - tile / tpp * tpp;
  if (pg < 0 || pg >= p.num_pages) return {-1, 0};
  const int64_t ph = pg * p.heads + h;
  return {(int)(ph * tpp + sub), (int)(ph * (tpp / tpq) + sub / tpq)};
}

// 8-token sub-tile `u` of (b, h) for stores whose quant block or page is 8 tokens (an odd
// multiple of 8): `data` in units of 8*D value bytes, `meta` the scale / zero entry of the
// quant block holding it; data = -1 when not backed by an allocated page.
template <bool PAGED>
__device__ __forceinline__ TileIndex sub_index(const DecodeParams& p, int b, int h, int row, int u) {
  const int token0 = 8 * u;
  if constexpr (PAGED) {
    const int lp = token0 / p.page_size;
    const int within = token0 - lp * p.page_size;
    if (lp >= p.table_cols) return {-1, 0};
    const int64_t pg = table_entry(p, b, lp);
    if (pg < 0 || pg >= p.num_pages) return {-1, 0};
    const int64_t ph = pg * p.heads + h;
    return {(int)(ph * (p.page_size / 8) + within / 8), (int)(ph * (p.page_size / p.quant_block) + within / p.quant_block)};
  } else {
    // the row's store holds n_blocks * quant_block tokens: an odd number of 8-token halves leaves the
    // last tile's second half past it (not backed; without this it would read past the store's end)
    if (token0 >= p.n_blocks * p.quant_block) return {-1, 0};
    return {row * p.n_blocks * (p.quant_block / 8) + u, row * p.n_blocks + token0 / p.quant_block};
  }
}

// Token mode: first token of tile `tile` of (b, h) in the value store (units of D bytes, the
// same index as its per-token scale / zero), -1 when not backed by an allocated page.
template <bool PAGED>
__device__ __forceinline__ int token_index(const DecodeParams& p, int b, int h, int row, int tile) {
  if constexpr (PAGED) {
    const int tpp = p.page_size / kTile;
    const int lp = tile / tpp;
    const int sub = tile - lp * tpp;
    if (lp >= p.table_cols) return -1;
    const int64_t pg = table_entry(p, b, lp);
    if (pg < 0 || pg >= p.num_pages) return -1;
    return (int)((pg * p.heads + h) * p.page_size + sub * kTile);
  } else {
    return row * p.n_blocks + tile * kTile;
  }
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// K/V bytes are read exactly once: non-temporal loads keep them from displacing the
// cache lines the rest of the GPU is using (measured: ~7% faster than plain loads).
__device__ __forceinline__ uint4 stream_load(const uint4* p) {
  const u32x4_t v = __builtin_nontemporal_load((const u32x4_t*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Paged-store parameters and checks (fs_decode.hip), shared with the tree verification entry
// point; row_kernel = false leaves the workgroup-size checks to the multi-query tree kernel.
int paged_params(DecodeParams& p, bool& tiled, const void* q, const int8_t* k_values, const float* k_scale,
                 const int16_t* k_zero, const int8_t* v_values, const float* v_scale, const int16_t* v_zero,
                 const void* block_table, int table_index_bytes, int64_t table_cols, const int64_t* lengths,
                 void* out, void* workspace, int64_t workspace_bytes, int batch, int nq, int heads, int head_dim,
                 int64_t num_pages, int page_size, int quant_block, int max_seq_len, float sm_scale, int split_tiles,
                 int max_splits, int waves_per_block, bool row_kernel = true, int vfmt = kVfInt8,
                 int per_channel = 0, void* merge_area = nullptr, int64_t merge_bytes = -1);

// The paged decode row kernel on `p` (fs_decode.hip).
int launch_paged_rows(const DecodeParams& p, int q_dtype, bool tiled, int waves_per_block, hipStream_t st);

}  // namespace fs
